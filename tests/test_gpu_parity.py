"""Parity of libmx's HIP kernels with the CPU oracle, through the C ABI, on device 0.

Bars: activation quantization and GET_ROWS bit-exact; products within max relative error 1e-3 of the oracle (largest
|difference| of a dst row over the largest |output| of that row). The kernels sum the same exact per-block integers as
the oracle and differ only in the order of the fp32 cross-block sum, so the observed error is ~1e-6; the test also
holds them to 1e-5 to catch a dropped term long before the 1e-3 bar would.
"""
import numpy as np
import pytest

import oracle as O
from helpers import bits_equal, dq_model, l2_rel, rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-3         # the parity bar
TIGHT = 2e-5       # what exact integer sums with an fp32 cross-block sum give


def dq_types(t, K):
    """Whether the dequantizing fp16 GEMM can take weights of type t and width K (Q8_0 K % 64, Q5_K / Q6_K K % 256)."""
    return (t == O.TYPE_Q8_0 and K % 64 == 0) or (t in (O.TYPE_Q5_K, O.TYPE_Q6_K) and K % 256 == 0)


def uses_dq(t, M, K, int8=False):
    """Whether MUL_MAT takes the dequantizing fp16 GEMM (its dispatch rule: past eight rows, Q5_K / Q6_K, and Q8_0
    where K is not a multiple of 128, which the int8 Q8_0 GEMM takes; int8: an int8 GEMM forced by the backend's
    options)."""
    return not int8 and M > 8 and dq_types(t, K) and not (t == O.TYPE_Q8_0 and K % 128 == 0)


def check_product(t, w, x, y, K, rounding=O.ROUND_REF, int8=False, y_ref=None, dq=None):
    """Parity of one product. The integer paths sum the oracle's exact per-block integers: held to TIGHT. The
    dequantizing fp16 GEMM rounds each operand to fp16 once: held to TOL against the oracle and to TIGHT against a
    model of exactly that rounding, which a dropped or misplaced term would miss by far more. dq: whether the product
    ran on the fp16 GEMM (None: as the dispatch rule picks)."""
    M = x.shape[0]
    if y_ref is None:
        y_ref = O.mul_mat(t, w, x, rounding=rounding)
    if uses_dq(t, M, K, int8) if dq is None else dq:
        assert rel_err(y, y_ref) <= TOL
        assert l2_rel(y, y_ref) <= TOL
        assert rel_err(y, dq_model(O, t, w, x, K, rounding)) <= TIGHT
    else:
        assert rel_err(y, y_ref) <= TIGHT
QTYPES = [O.TYPE_Q8_0, O.TYPE_Q4_K, O.TYPE_Q5_K, O.TYPE_Q6_K]
FTYPES = [O.TYPE_F16, O.TYPE_F32]
NAMES = {O.TYPE_Q8_0: "q8_0", O.TYPE_Q4_K: "q4_K", O.TYPE_Q5_K: "q5_K", O.TYPE_Q6_K: "q6_K", O.TYPE_F16: "f16",
         O.TYPE_F32: "f32"}


def weights(t, N, K, seed, std=0.02):
    return O.quantize_chunk(t, O.fill_normal(seed, N, K, 0.0, std))


def acts(seed, M, K):
    return O.fill_normal(seed, M, K, 0.0, 1.0)


def special_rows(K):
    """Rows that exercise the quantizers' edge cases."""
    rows = []
    rows.append(np.zeros(K, np.float32))                                   # all-zero blocks: d = 0, q = 0
    rows.append(np.full(K, 0.75, np.float32))                              # constant blocks: q = +-127
    r = np.zeros(K, np.float32)
    r[0::32] = 127.0
    r[1::32] = 2.5                                                         # REF rounds 2.5 -> 3, X86 -> 2
    r[2::32] = -2.5
    r[3::32] = 0.5
    rows.append(r)
    rows.append((np.arange(K, dtype=np.float32) % 7 - 3) * np.float32(1e-6))  # fp16-subnormal scales
    t = np.zeros(K, np.float32)
    t[5::256] = -3.0
    t[9::256] = 3.0                                                        # Q8_K tie on |max|: the first (-3) wins
    t[100::256] = 1.0
    rows.append(t)
    rows.append(-np.abs(acts(11, 1, K)[0]))                                # one-signed
    return np.stack(rows).astype(np.float32)


# --------------------------------------------------------------------------------------------- activation quantizers
@pytest.mark.parametrize("qt", [O.TYPE_Q8_0, O.TYPE_Q8_1, O.TYPE_Q8_K])
@pytest.mark.parametrize("rounding", [O.ROUND_REF, O.ROUND_X86])
def test_quantize_act_bit_exact(mx, be, qt, rounding):
    if qt == O.TYPE_Q8_K and rounding == O.ROUND_X86:
        pytest.skip("Q8_K has a single rounding")
    K = 4096
    x = np.concatenate([acts(0xAC700001, 9, K), special_rows(K), acts(3, 2, K) * np.float32(1e4)])
    tx = be.tensor(mx.F32, (K, x.shape[0]), x)
    out = be.quantize_act(qt, rounding, tx, K, x.shape[0])
    be.sync()
    got = out.get_bytes()[: O.row_size(qt, K) * x.shape[0]].reshape(x.shape[0], -1)
    want = O.quantize_rows(qt, x, rounding)
    assert np.array_equal(got, want), f"rows differing: {np.nonzero((got != want).any(axis=1))[0]}"


# ------------------------------------------------------------------------------------------------ device layout
@pytest.mark.parametrize("t", QTYPES, ids=lambda t: NAMES[t])
def test_tensor_set_get_roundtrip(mx, be, t):
    K, N = 512, 37
    w = weights(t, N, K, 0x5EED0100 + t).reshape(-1)
    T = be.tensor(t, (K, N))
    cuts = [0, 1, 35, 36, 143, 500, 1000, 2049, len(w)]   # pieces at offsets that split blocks and fields
    for a, b in zip(cuts[:-1], cuts[1:]):
        T.set(w[a:b], offset=a)
    assert np.array_equal(T.get_bytes(), w)
    assert np.array_equal(T.get_bytes(offset=37, size=301), w[37:338])
    T.set(np.zeros(50, np.uint8), offset=211)
    ref = w.copy()
    ref[211:261] = 0
    assert np.array_equal(T.get_bytes(), ref)


def test_tensor_set_out_of_range(mx, be):
    T = be.tensor(mx.Q8_0, (64, 2))
    with pytest.raises(mx.MxError) as e:
        T.set(np.zeros(10, np.uint8), offset=T.nbytes - 5)
    assert e.value.code == mx.INVALID


# ---------------------------------------------------------------------------------------------------- GET_ROWS
@pytest.mark.parametrize("t", QTYPES, ids=lambda t: NAMES[t])
def test_get_rows_bit_exact(mx, be, t):
    K, R = 1024, 50
    table = weights(t, R, K, 0x5EED0200 + t)
    ids = np.array([0, 49, 7, 7, 23, 1], np.int32)
    T = be.tensor(t, (K, R), table)
    I = be.tensor(mx.I32, (len(ids),), ids)
    D = be.tensor(mx.F32, (K, len(ids)))
    be.get_rows(T, I, D)
    be.sync()
    got = D.numpy().reshape(len(ids), K)
    assert bits_equal(got, O.get_rows(t, table, K, ids))


@pytest.mark.parametrize("t", QTYPES, ids=lambda t: NAMES[t])
def test_get_rows_3d(mx, be, t):
    # src0 [K, R, 3], ids [n, 3]: matrix i11 of the table for the ids of column i11 (ggml_get_rows broadcast rule)
    K, R, B, n = 256, 10, 3, 4
    table = weights(t, R * B, K, 0x5EED0300 + t)
    ids = np.array([[0, 9, 3, 3], [1, 1, 2, 8], [9, 0, 5, 4]], np.int32)
    T = be.tensor(t, (K, R, B), table)
    I = be.tensor(mx.I32, (n, B), ids)
    D = be.tensor(mx.F32, (K, n, B))
    be.get_rows(T, I, D)
    be.sync()
    got = D.numpy().reshape(B, n, K)
    for b in range(B):
        want = O.get_rows(t, table[b * R:(b + 1) * R], K, ids[b])
        assert bits_equal(got[b], want)


def test_get_rows_index_out_of_range(mx, be):
    K, R = 256, 8
    T = be.tensor(mx.Q8_0, (K, R), weights(O.TYPE_Q8_0, R, K, 5))
    I = be.tensor(mx.I32, (2,), np.array([3, R], np.int32))
    D = be.tensor(mx.F32, (K, 2))
    be.get_rows(T, I, D)
    with pytest.raises(mx.MxError) as e:
        be.sync()
    assert e.value.code == mx.INVALID
    assert np.all(D.numpy().reshape(2, K)[1] == 0)
    be.sync()  # the error word was cleared


def test_get_rows_more_rows_than_workgroups(mx, be):
    """140,000 output rows on a grid of at most 65,536 workgroups: each workgroup takes rows i, i + 65,536, ...; an
    out-of-range id met on a workgroup's second row is zeroed and reported like one on its first."""
    K, R, n = 64, 300, 140_000
    table = weights(O.TYPE_Q8_0, R, K, 0x5EED0400)
    ids = np.random.default_rng(11).integers(0, R, n).astype(np.int32)
    T = be.tensor(mx.Q8_0, (K, R), table)
    I = be.tensor(mx.I32, (n,), ids)
    D = be.tensor(mx.F32, (K, n))
    be.get_rows(T, I, D)
    be.sync()
    assert bits_equal(D.numpy().reshape(n, K), O.get_rows(O.TYPE_Q8_0, table, K, ids))
    bad = ids.copy()
    bad[70_000] = R
    I2 = be.tensor(mx.I32, (n,), bad)
    be.get_rows(T, I2, D)
    with pytest.raises(mx.MxError) as e:
        be.sync()
    assert e.value.code == mx.INVALID
    got = D.numpy().reshape(n, K)
    assert np.all(got[70_000] == 0)
    keep = np.arange(n) != 70_000
    assert bits_equal(got[keep], O.get_rows(O.TYPE_Q8_0, table, K, ids[keep]))
    be.sync()


# ------------------------------------------------------------------------------------------------------ MUL_MAT
def run_mul_mat(mx, be, t, w, x, K, N):
    M = x.shape[0]
    W = be.tensor(t, (K, N), w)
    X = be.tensor(mx.F32, (K, M), x)
    Y = be.tensor(mx.F32, (N, M))
    be.mul_mat(W, X, Y)
    be.sync()
    return Y.numpy().reshape(M, N)


@pytest.mark.parametrize("t", QTYPES, ids=lambda t: NAMES[t])
@pytest.mark.parametrize("M", [1, 2, 3, 5, 8, 11])
def test_mul_mat_small_m(mx, be, t, M):
    K = 1536 if t != O.TYPE_Q8_0 else 1056
    N = 301
    w = weights(t, N, K, 0x5EED0400 + t)
    x = acts(0xAC700400 + M, M, K)
    y = run_mul_mat(mx, be, t, w, x, K, N)
    if uses_dq(t, M, K):  # past eight columns Q8_0 at K % 128 != 0 and Q6_K take the fp16 GEMM
        check_product(t, w, x, y, K)
        return
    assert rel_err(y, O.mul_mat(t, w, x)) <= TIGHT
    assert rel_err(y, O.mul_mat(t, w, x, exact=True)) <= TIGHT


@pytest.mark.parametrize("t", QTYPES, ids=lambda t: NAMES[t])
@pytest.mark.parametrize("K", [256, 2048, 6144])
def test_mul_mat_matvec_k(mx, be, t, K):
    N = 130
    w = weights(t, N, K, 0x5EED0500 + K + t)
    x = acts(0xAC700500 + K, 1, K)
    assert rel_err(run_mul_mat(mx, be, t, w, x, K, N), O.mul_mat(t, w, x)) <= TIGHT


def test_mul_mat_config1(mx, be):
    """Single MUL_MAT, batch 1: W 3072 x 1024 from N(0, 0.02) quantized to Q8_0 by quantize_row_q8_0_ref; x 1 x 1024
    from N(0, 1); y 1 x 3072."""
    K, N = 1024, 3072
    w = weights(O.TYPE_Q8_0, N, K, 0x5EED0010)
    x = acts(0xAC700001, 1, K)
    y = run_mul_mat(mx, be, O.TYPE_Q8_0, w, x, K, N)
    y_ref = O.mul_mat(O.TYPE_Q8_0, w, x)
    assert rel_err(y, y_ref) <= TIGHT
    assert l2_rel(y, y_ref) <= TIGHT


@pytest.mark.parametrize("t", [O.TYPE_Q8_0, O.TYPE_Q4_K, O.TYPE_Q6_K], ids=lambda t: NAMES[t])
@pytest.mark.parametrize("M", [1, 3])
def test_mul_mat_many_row_blocks(mx, be, t, M):
    """40,001 rows (2,501 blocks of 16, the last ragged), plain and with the fused residual ADD (bit for bit the
    separate ADD)."""
    K, N = 256, 40_001
    w = weights(t, N, K, 0x5EED1100 + t + M)
    x = acts(0xAC701100 + M, M, K)
    y = run_mul_mat(mx, be, t, w, x, K, N)
    assert rel_err(y, O.mul_mat(t, w, x)) <= TIGHT
    r = acts(0xAC701180 + M, M, N)
    W = be.tensor(t, (K, N), w)
    X = be.tensor(mx.F32, (K, M), x)
    R = be.tensor(mx.F32, (N, M), r)
    be.mul_mat_fused([W], X, [R], residual=[R])
    be.sync()
    got = R.numpy().reshape(M, N)
    assert bits_equal(got, (r.reshape(M, N) + y.reshape(M, N)).astype(np.float32))


def test_mul_mat_output_head_full_shape(mx, be):
    """The 0.6B shape's tied output head at its full size: 151,936 x 1024 Q8_0 (166 MB, 9,496 row blocks) on one
    column, as the decode step's last product runs it."""
    K, N = 1024, 151_936
    w = mx.quantize_normal(O.TYPE_Q8_0, 0x5EED4100, N, K, 0.02)
    x = acts(0xAC704100, 1, K)
    assert rel_err(run_mul_mat(mx, be, O.TYPE_Q8_0, w, x, K, N), O.mul_mat(O.TYPE_Q8_0, w, x)) <= TIGHT


@pytest.mark.parametrize("t", QTYPES, ids=lambda t: NAMES[t])
def test_mul_mat_x86_rounding(mx, be, t):
    K, N, M = 512, 64, 3
    w = weights(t, N, K, 0x5EED0600 + t)
    x = np.concatenate([acts(0xAC700600, M, K), special_rows(K)[2:3]])
    be.set_rounding(mx.ROUND_X86)
    try:
        y = run_mul_mat(mx, be, t, w, x, K, N)
    finally:
        be.set_rounding(mx.ROUND_REF)
    assert rel_err(y, O.mul_mat(t, w, x, rounding=O.ROUND_X86)) <= TIGHT


@pytest.mark.parametrize("path", ["int8", "fp16"])
def test_gemm_q8_0_x86_rounding(mx, be, path):
    """The x86 activation rounding (rint of x * 127 / amax) through both Q8_0 GEMMs, 40 rows with a special row:
    the int8 GEMM to TIGHT of the oracle under the same rounding, the fp16 one to its model of that rounding."""
    t, K, N = O.TYPE_Q8_0, 512, 200
    w = weights(t, N, K, 0x5EED0610)
    x = np.concatenate([acts(0xAC700610, 39, K), special_rows(K)[2:3]])
    be.set_rounding(mx.ROUND_X86)
    try:
        with be.options(gemm_q8_0=Q8_PATHS[path]):
            y = run_mul_mat(mx, be, t, w, x, K, N)
    finally:
        be.set_rounding(mx.ROUND_REF)
    check_product(t, w, x, y, K, rounding=O.ROUND_X86, dq=path == "fp16")
    # the REF rounding gives other quants for this row set: a kernel that ignored the mode would miss
    y_ref = O.mul_mat(t, w, x, rounding=O.ROUND_REF)
    assert not np.array_equal(O.mul_mat(t, w, x, rounding=O.ROUND_X86), y_ref)


@pytest.mark.parametrize("t", QTYPES, ids=lambda t: NAMES[t])
def test_mul_mat_batched_broadcast(mx, be, t):
    # src0 [K, N, 2, 1], src1 [K, M, 4, 2]: r2 = 2, r3 = 2 (ggml broadcast of src0 over src1's batch axes)
    K, N, M = 256, 40, 2
    w = weights(t, N * 2, K, 0x5EED0700 + t)
    x = acts(0xAC700700, M * 4 * 2, K).reshape(2, 4, M, K)
    W = be.tensor(t, (K, N, 2, 1), w)
    X = be.tensor(mx.F32, (K, M, 4, 2), x)
    Y = be.tensor(mx.F32, (N, M, 4, 2))
    be.mul_mat(W, X, Y)
    be.sync()
    y = Y.numpy()
    for i3 in range(2):
        for i2 in range(4):
            wm = w[(i2 // 2) * N:(i2 // 2 + 1) * N]
            assert rel_err(y[i3, i2], O.mul_mat(t, wm, x[i3, i2])) <= TIGHT


@pytest.mark.parametrize("t", QTYPES, ids=lambda t: NAMES[t])
def test_mul_mat_group(mx, be, t):
    # q / k / v of one layer share src1: one launch, three results
    K, M = 1024, 2
    Ns = [256, 128, 128]
    ws = [weights(t, n, K, 0x5EED0800 + i + t) for i, n in enumerate(Ns)]
    x = acts(0xAC700800, M, K)
    W = [be.tensor(t, (K, n), w) for n, w in zip(Ns, ws)]
    X = be.tensor(mx.F32, (K, M), x)
    Y = [be.tensor(mx.F32, (n, M)) for n in Ns]
    be.mul_mat_group(W, X, Y)
    be.sync()
    for n, w, yt in zip(Ns, ws, Y):
        assert rel_err(yt.numpy().reshape(M, n), O.mul_mat(t, w, x)) <= TIGHT


def test_supports_op(mx, be):
    W = be.tensor(mx.Q4_K, (300 // 256 * 256 + 256, 4))
    X = be.tensor(mx.F32, (W.ne[0], 1))
    Y = be.tensor(mx.F32, (4, 1))
    assert be.supports(mx.OP_MUL_MAT, W, X, None, Y)
    Xbad = be.tensor(mx.F32, (W.ne[0] - 256, 1))
    assert not be.supports(mx.OP_MUL_MAT, W, Xbad, None, Y)
    F = be.tensor(mx.F32, (W.ne[0], 4))
    assert be.supports(mx.OP_MUL_MAT, F, X, None, Y)       # F32 weights: the float mat-vec
    H = be.tensor(mx.F16, (W.ne[0] - 4, 4))
    Xh = be.tensor(mx.F32, (W.ne[0] - 4, 1))
    assert not be.supports(mx.OP_MUL_MAT, H, Xh, None, Y)  # F16 rows of whole 8-element loads only


# --------------------------------------------------------------------------------------------------- MUL_MAT_ID
def mmid_uses_dq(t, K, npairs, E, kernel=0, matvec_pairs=16):
    """Whether MUL_MAT_ID takes the dequantizing fp16 GEMM over chunks of each expert's pairs (its dispatch rule:
    Q8_0 / Q5_K / Q6_K experts, more pairs than the mat-vec launch takes, on average at least one (Q8_0) or three
    (K-quants) pairs per expert, or the GEMM forced; never when the experts kernel is forced)."""
    if npairs <= matvec_pairs or kernel == 1 or not dq_types(t, K):
        return False
    return kernel == 2 or npairs >= (1 if t == O.TYPE_Q8_0 else 3) * E


def mmid_dq_model(t, w, x, ids, K):
    """dq_model for each expert's pairs: what the dequantizing GEMM computes for routed rows."""
    T, n_ids = ids.shape
    B = x.shape[1]
    y = np.zeros((T, n_ids, w.shape[1]))
    for e in np.unique(ids):
        tt, ss = np.nonzero(ids == e)
        y[tt, ss] = dq_model(O, t, w[e], x[tt, ss % B], K)
    return y


class MmidRef:
    """The inputs of one MUL_MAT_ID and the bar its path is held to: the integer paths to TIGHT against the oracle;
    the dequantizing fp16 GEMM to TOL against the oracle and to TIGHT against a model of its roundings."""

    def __init__(self, t, w, x, ids, K, dq):
        self.t, self.w, self.x, self.ids, self.K, self.dq = t, w, x, ids, K, dq

    def check(self, y, what=""):
        y_ref = O.mul_mat_id(self.t, self.w, self.x, self.ids)
        if self.dq:
            assert rel_err(y, y_ref) <= TOL, what
            assert l2_rel(y, y_ref) <= TOL, what
            assert rel_err(y, mmid_dq_model(self.t, self.w, self.x, self.ids, self.K)) <= TIGHT, what
        else:
            assert rel_err(y, y_ref) <= TIGHT, what


def mmid_case(mx, be, t, E, K, N, n_ids, T, bcast, seed, skew=0.0, ids=None):
    w = weights(t, E * N, K, seed).reshape(E, N, -1)
    B = 1 if bcast else n_ids
    x = acts(seed + 1, T * B, K).reshape(T, B, K)
    if ids is None:
        rng = np.random.default_rng(seed)
        logits = rng.standard_normal((T, E))
        logits[:, :n_ids] += skew  # a large skew sends most tokens to the same experts
        ids = np.argsort(-logits, axis=1)[:, :n_ids].astype(np.int32)
    Wt = be.tensor(t, (K, N, E), w.reshape(E * N, -1))
    Xt = be.tensor(mx.F32, (K, B, T), x)
    It = be.tensor(mx.I32, (n_ids, T), ids)
    Yt = be.tensor(mx.F32, (N, n_ids, T))
    be.mul_mat_id(Wt, Xt, It, Yt)
    be.sync()
    y = Yt.numpy().reshape(T, n_ids, N)
    dq = mmid_uses_dq(t, K, n_ids * T, E, be.get_option("mmid_kernel"), be.get_option("mmid_matvec_pairs"))
    return y, MmidRef(t, w, x, ids, K, dq)


@pytest.mark.parametrize("t", QTYPES, ids=lambda t: NAMES[t])
@pytest.mark.parametrize("T", [1, 3, 16, 40])
@pytest.mark.parametrize("bcast", [True, False], ids=["b_bcast", "b_per_slot"])
def test_mul_mat_id(mx, be, t, T, bcast):
    y, ref = mmid_case(mx, be, t, E=8, K=512, N=96, n_ids=2, T=T, bcast=bcast, seed=0x5EED0900 + T + t)
    ref.check(y)


@pytest.mark.parametrize("t", QTYPES, ids=lambda t: NAMES[t])
@pytest.mark.parametrize("skew", [0.0, 3.0], ids=["spread", "skewed"])
def test_mul_mat_id_many_pairs(mx, be, t, skew):
    """Experts with more than 16 pairs (several tiles, a ragged last one) and N not a multiple of the column tile."""
    y, ref = mmid_case(mx, be, t, E=16, K=1024, N=200, n_ids=4, T=70, bcast=False, seed=0x5EED0A00 + t, skew=skew)
    ref.check(y)


@pytest.mark.parametrize("t", QTYPES, ids=lambda t: NAMES[t])
@pytest.mark.parametrize("chunk", [0, 16], ids=["chunk_picked", "chunk16"])
def test_mul_mat_id_chunk_edges(mx, be, t, chunk):
    """Experts with exactly 16, 17, 32, 33 and 70 pairs (one or two 16-row tiles per chunk, a chunk of one pair)
    and none, at K = 2048 (the longest K the Q4_K expert kernel keeps in LDS) with b broadcast over the slots; for
    Q4_K in chunks of 32 (as picked here) and of 16 (the kernel form without a second tile)."""
    counts = [16, 17, 0, 32, 33, 70]
    ids = np.concatenate([np.full(c, e, np.int32) for e, c in enumerate(counts)])
    np.random.default_rng(7).shuffle(ids)
    with be.options(mmid_chunk=chunk):
        y, ref = mmid_case(mx, be, t, E=len(counts), K=2048, N=136, n_ids=1, T=len(ids), bcast=True,
                           seed=0x5EED0B00 + t, ids=ids.reshape(-1, 1))
    ref.check(y)


@pytest.mark.parametrize("t", QTYPES, ids=lambda t: NAMES[t])
def test_mul_mat_id_past_held_pairs(mx, be, t):
    """2,400 (token, slot) pairs: the bucketing pass keeps a thread's first eight pairs' experts in registers (2,048
    pairs over its 256 threads) and reads the rest again for its second pass."""
    y, ref = mmid_case(mx, be, t, E=8, K=256, N=40, n_ids=4, T=600, bcast=True, seed=0x5EED0F00 + t)
    ref.check(y)


@pytest.mark.parametrize("t", QTYPES, ids=lambda t: NAMES[t])
def test_mul_mat_id_long_rows(mx, be, t):
    """K = 4096, past what the grouped Q4_K product keeps in LDS: for Q4_K the experts kernel by default, in one pass
    (20 tokens over 16 experts) and in several passes of eight pairs (40 tokens over 4 experts, ~20 pairs each); the
    other types on the fp16 GEMM over chunks of each expert's pairs, at the same shapes."""
    for E, T, seed in ((16, 20, 0x5EED0E00), (4, 40, 0x5EED0E40)):
        y, ref = mmid_case(mx, be, t, E=E, K=4096, N=72, n_ids=2, T=T, bcast=False, seed=seed + t)
        ref.check(y, f"E {E}, T {T}")


@pytest.mark.parametrize("t", QTYPES, ids=lambda t: NAMES[t])
def test_mul_mat_id_moe_layer_shape(mx, be, t):
    """The drama3-like layer's down product (64 experts, top-4 of 64 tokens, K = 1536, b per slot) on 520 of its
    2048 output rows."""
    y, ref = mmid_case(mx, be, t, E=64, K=1536, N=520, n_ids=4, T=64, bcast=False, seed=0x5EED0C00 + t)
    ref.check(y)


@pytest.mark.parametrize("t", QTYPES, ids=lambda t: NAMES[t])
@pytest.mark.parametrize("T", [2, 16, 40])
def test_mul_mat_id_group(mx, be, t, T):
    """Gate and up experts over the same rows and ids in one call (mx_mul_mat_id_group): each product the same bits as
    its own mx_mul_mat_id -- one mat-vec launch for both at 2 tokens, the grouped product's two forms at 16 and 40
    (Q4_K), one launch of the fp16 GEMM over each expert's chunks for both products after a shared prep (Q8_0, Q5_K,
    Q6_K) -- and within its path's bar against the oracle."""
    E, K, N, n_ids = 16, 1024, 200, 4
    seed = 0x5EED0D00 + 64 * T + t
    wg = weights(t, E * N, K, seed).reshape(E, N, -1)
    wu = weights(t, E * N, K, seed + 1).reshape(E, N, -1)
    x = acts(seed + 2, T, K).reshape(T, 1, K)
    logits = np.random.default_rng(seed).standard_normal((T, E))
    ids = np.argsort(-logits, axis=1)[:, :n_ids].astype(np.int32)
    Wg = be.tensor(t, (K, N, E), wg.reshape(E * N, -1))
    Wu = be.tensor(t, (K, N, E), wu.reshape(E * N, -1))
    Xt = be.tensor(mx.F32, (K, 1, T), x)
    It = be.tensor(mx.I32, (n_ids, T), ids)
    Ys = [be.tensor(mx.F32, (N, n_ids, T)) for _ in range(2)]
    Yg = [be.tensor(mx.F32, (N, n_ids, T)) for _ in range(2)]
    be.mul_mat_id(Wg, Xt, It, Ys[0])
    be.mul_mat_id(Wu, Xt, It, Ys[1])
    be.mul_mat_id_group([Wg, Wu], Xt, It, Yg)
    be.sync()
    dq = mmid_uses_dq(t, K, n_ids * T, E)
    for a, b, w in zip(Ys, Yg, (wg, wu)):
        assert np.array_equal(a.numpy(), b.numpy())
        MmidRef(t, w, x, ids, K, dq).check(b.numpy().reshape(T, n_ids, N))


_MOE_FULL = {}


def moe_full_weights(mx):
    """The full-shape MoE layer's gate, up and down experts (Q4_K from N(0, 0.02)), quantized once per run."""
    if not _MOE_FULL:
        E, H, F = 64, 2048, 1536
        _MOE_FULL["w"] = tuple(mx.quantize_normal(O.TYPE_Q4_K, 0x5EED4000 + i, E * n, k, 0.02).reshape(E, n, -1)
                               for i, (n, k) in enumerate(((F, H), (F, H), (H, F))))
    return _MOE_FULL["w"]


@pytest.mark.parametrize("T", [1, 16, 256])
def test_moe_layer_full_shape(mx, be, T):
    """The drama3-like MoE FFN at its full shape (text-model.cpp:198-221): 64 Q4_K experts, hidden 2048, expert FFN 1536,
    top-4 of N(0, 1) router logits per token, T = 1 / 16 / 256 tokens -- the gate and up experts as one group over the
    shared rows (the launch the layer spends most of its time in at 256 tokens: 1,024 pairs over all 64 experts) and
    the down experts over per-slot rows. The kernels compute every output row; every fifth row of each expert (rows in
    every column tile) is held to the oracle on the same bytes."""
    E, H, F, n_ids = 64, 2048, 1536, 4
    t = O.TYPE_Q4_K
    seed = 0x5EED4000 + T
    wg, wu, wd = moe_full_weights(mx)
    x = acts(seed + 3, T, H).reshape(T, 1, H)
    logits = O.fill_normal(seed + 4, T, E)
    ids = np.argsort(-logits, axis=1, kind="stable")[:, :n_ids].astype(np.int32)
    Wg, Wu = be.tensor(t, (H, F, E), wg.reshape(E * F, -1)), be.tensor(t, (H, F, E), wu.reshape(E * F, -1))
    Wd = be.tensor(t, (F, H, E), wd.reshape(E * H, -1))
    Xt, It = be.tensor(mx.F32, (H, 1, T), x), be.tensor(mx.I32, (n_ids, T), ids)
    Yg, Yu = be.tensor(mx.F32, (F, n_ids, T)), be.tensor(mx.F32, (F, n_ids, T))
    be.mul_mat_id_group([Wg, Wu], Xt, It, [Yg, Yu])
    be.sync()
    rows = np.arange(0, F, 5)
    for Y, w in ((Yg, wg), (Yu, wu)):
        got = Y.numpy().reshape(T, n_ids, F)[:, :, rows]
        assert rel_err(got, O.mul_mat_id(t, np.ascontiguousarray(w[:, rows]), x, ids)) <= TIGHT
    act = acts(seed + 5, T * n_ids, F).reshape(T, n_ids, F)
    At, Yd = be.tensor(mx.F32, (F, n_ids, T), act), be.tensor(mx.F32, (H, n_ids, T))
    be.mul_mat_id(Wd, At, It, Yd)
    be.sync()
    rows = np.arange(0, H, 5)
    got = Yd.numpy().reshape(T, n_ids, H)[:, :, rows]
    assert rel_err(got, O.mul_mat_id(t, np.ascontiguousarray(wd[:, rows]), act, ids)) <= TIGHT


def test_mul_mat_id_group_refusals(mx, be):
    K, N, E, T = 256, 32, 4, 3
    W = be.tensor(mx.Q8_0, (K, N, E), weights(O.TYPE_Q8_0, E * N, K, 11))
    W2 = be.tensor(mx.Q8_0, (K, N + 32, E), weights(O.TYPE_Q8_0, E * (N + 32), K, 12))
    X = be.tensor(mx.F32, (K, 1, T), acts(13, T, K))
    I = be.tensor(mx.I32, (2, T), np.array([[0, 1], [2, 3], [1, 0]], np.int32))
    Y = [be.tensor(mx.F32, (N, 2, T)) for _ in range(2)]
    Y2 = be.tensor(mx.F32, (N + 32, 2, T))
    with pytest.raises(mx.MxError) as e:  # experts of another shape
        be.mul_mat_id_group([W, W2], X, I, [Y[0], Y2])
    assert e.value.code == mx.UNSUPPORTED
    with pytest.raises(mx.MxError) as e:  # more than four
        be.mul_mat_id_group([W] * 5, X, I, [Y[0]] * 5)
    assert e.value.code == mx.INVALID


def test_mul_mat_id_bad_expert(mx, be):
    K, N, E = 256, 32, 4
    Wt = be.tensor(mx.Q8_0, (K, N, E), weights(O.TYPE_Q8_0, E * N, K, 9))
    Xt = be.tensor(mx.F32, (K, 1, 2), acts(10, 2, K))
    It = be.tensor(mx.I32, (2, 2), np.array([[0, 1], [3, E]], np.int32))
    Yt = be.tensor(mx.F32, (N, 2, 2))
    be.mul_mat_id(Wt, Xt, It, Yt)
    with pytest.raises(mx.MxError) as e:
        be.sync()
    assert e.value.code == mx.INVALID
    be.sync()


# ------------------------------------------------------------------------------------------------------- graphs
def test_graph_replay_matches_eager(mx, be):
    K, N, R = 1024, 512, 16
    tab = weights(O.TYPE_Q8_0, R, K, 21)
    w = weights(O.TYPE_Q8_0, N, K, 22)
    T = be.tensor(mx.Q8_0, (K, R), tab)
    W = be.tensor(mx.Q8_0, (K, N), w)
    I = be.tensor(mx.I32, (1,), np.array([3], np.int32))
    X = be.tensor(mx.F32, (K, 1))
    Y = be.tensor(mx.F32, (N, 1))
    be.get_rows(T, I, X)
    be.mul_mat(W, X, Y)
    be.sync()
    be.graph_begin()
    be.get_rows(T, I, X)
    be.mul_mat(W, X, Y)
    g = be.graph_end()
    try:
        for tok in [5, 0, 15, 5]:
            I.set(np.array([tok], np.int32))
            be.graph_launch(g)
            be.sync()
            x_ref = O.get_rows(O.TYPE_Q8_0, tab, K, np.array([tok], np.int32))
            assert bits_equal(X.numpy().reshape(1, K), x_ref)
            assert rel_err(Y.numpy().reshape(1, N), O.mul_mat(O.TYPE_Q8_0, w, x_ref)) <= TIGHT
    finally:
        be.graph_free(g)


# ----------------------------------------------------------------------------------------------- MUL_MAT, M > 8
Q8_PATHS = {"int8": 0, "fp16": 2}  # the Q8_0 GEMM option: as picked (the int8 GEMM), the fp16 GEMM forced


@pytest.mark.parametrize("t", [O.TYPE_Q8_0, O.TYPE_Q4_K, O.TYPE_Q6_K], ids=lambda t: NAMES[t])
def test_gemm_rows_past_grid_y(mx, be, t):
    """66,000 rows, more than a grid's y dimension holds (65,535): the activation passes put the rows on x."""
    M, N, K = 66000, 40, 256
    w = weights(t, N, K, 0x5EED1700 + t)
    x = acts(0xAC701700, M, K)
    y = run_mul_mat(mx, be, t, w, x, K, N)
    check_product(t, w, x, y, K)


# (type, Q8_0 option, rows, widths, K): the int8 Q8_0 GEMM split four ways (28 rows, a group) and on 64 x 128 tiles
# unsplit (130 rows x 2 x 3000: 564 tiles of 64 x 128), the fp16 GEMM split (Q8_0 forced, Q6_K), the Q4_K GEMM
GRAPH_CASES = {"q8_0_int8_split": (O.TYPE_Q8_0, 0, 28, [200, 64, 72], 2048),
               "q8_0_int8_wide": (O.TYPE_Q8_0, 0, 130, [3000, 3000], 1024),
               "q8_0_fp16_split": (O.TYPE_Q8_0, 2, 28, [200, 64, 72], 2048),
               "q6_K_fp16": (O.TYPE_Q6_K, 0, 40, [1000], 4096),
               "q4_K": (O.TYPE_Q4_K, 0, 130, [1024, 512], 2048)}


@pytest.mark.parametrize("case", list(GRAPH_CASES))
def test_gemm_graph_replays(mx, be, case):
    """A prefill group recorded into a graph and replayed three times, with eager products and the outputs
    overwritten between the replays: every replay gives the eager run's bits (the split partials and their reduce
    included), and the eager run is held to the oracle."""
    t, q8, M, Ns, K = GRAPH_CASES[case]
    ws = [weights(t, n, K, 0x5EED1600 + 13 * i + t) for i, n in enumerate(Ns)]
    x = acts(0xAC701600 + M, M, K)
    W = [be.tensor(t, (K, n), w) for n, w in zip(Ns, ws)]
    X = be.tensor(mx.F32, (K, M), x)
    Y = [be.tensor(mx.F32, (n, M)) for n in Ns]
    other_w = be.tensor(t, (K, 96), weights(t, 96, K, 0x5EED1650 + t))
    other_y = be.tensor(mx.F32, (96, M))
    with be.options(gemm_q8_0=q8):
        be.mul_mat_group(W, X, Y)
        be.sync()
        eager = [yt.numpy().reshape(M, n).copy() for n, yt in zip(Ns, Y)]
        for w, y in zip(ws, eager):
            check_product(t, w, x, y, K, dq=None if t != O.TYPE_Q8_0 else q8 == 2)
        be.mul_mat(other_w, X, other_y)  # (the scratch at its largest before the recording)
        be.graph_begin()
        be.mul_mat_group(W, X, Y)
        g = be.graph_end()
        try:
            for rep in range(3):
                for yt, n in zip(Y, Ns):
                    yt.set(np.full((M, n), np.nan, np.float32))
                be.mul_mat(other_w, X, other_y)  # eager work between the replays, on the same scratch
                be.sync()
                be.graph_launch(g)
                be.sync()
                for n, yt, y in zip(Ns, Y, eager):
                    assert bits_equal(yt.numpy().reshape(M, n), y), f"replay {rep}"
        finally:
            be.graph_free(g)


@pytest.mark.parametrize("path", list(Q8_PATHS))
@pytest.mark.parametrize("M,N,K", [(9, 100, 1024), (64, 256, 2048), (130, 333, 1024), (512, 2048, 2048),
                                   (100, 64, 6144), (650, 4500, 512), (300, 8100, 256), (520, 8200, 256),
                                   (200, 300, 1152)])
def test_mul_mat_gemm_q8_0(mx, be, M, N, K, path):
    """Both Q8_0 GEMMs. Short blocks split K (9 and 64 rows; 100 rows over K = 6144); on the fp16 GEMM three take
    128 x 128 tiles unsplit with ragged rows and columns (216, 192 and 325 workgroups: the last more than the CUs);
    K = 256 and 512 have two and four stages of 128, fewer than the int8 GEMM's 64 x 64 copy ring holds; K = 1152 ends
    one 128-wide stage past a 1024-element piece of the activation pass; 520 x 8200 takes the int8 GEMM's 64 x 128
    tile (585 of them: its two-stage ring)."""
    t = O.TYPE_Q8_0
    w = weights(t, N, K, 0x5EED0A00 + M + N)
    x = acts(0xAC700A00 + M, M, K)
    with be.options(gemm_q8_0=Q8_PATHS[path]):
        y = run_mul_mat(mx, be, t, w, x, K, N)
    check_product(t, w, x, y, K, dq=path == "fp16")


@pytest.mark.parametrize("path", list(Q8_PATHS))
def test_mul_mat_gemm_group_q8_0_split(mx, be, path):
    """A short block (28 rows) through either grouped Q8_0 GEMM: K is split over several workgroups per tile and the
    partial sums of the three products are added by one reduce pass; a second run gives the same bits."""
    t, K, M = O.TYPE_Q8_0, 2048, 28
    Ns = [200, 64, 72]
    ws = [weights(t, n, K, 0x5EED0E00 + i) for i, n in enumerate(Ns)]
    x = acts(0xAC700E00, M, K)
    W = [be.tensor(t, (K, n), w) for n, w in zip(Ns, ws)]
    X = be.tensor(mx.F32, (K, M), x)
    Y = [be.tensor(mx.F32, (n, M)) for n in Ns]
    with be.options(gemm_q8_0=Q8_PATHS[path]):
        be.mul_mat_group(W, X, Y)
        be.sync()
        first = [yt.numpy().reshape(M, n).copy() for n, yt in zip(Ns, Y)]
        for n, w, y in zip(Ns, ws, first):
            check_product(t, w, x, y, K, dq=path == "fp16")
        be.mul_mat_group(W, X, Y)
        be.sync()
    for n, yt, y in zip(Ns, Y, first):
        assert bits_equal(yt.numpy().reshape(M, n), y)


@pytest.mark.parametrize("t,M,Ns,K,q8", [(O.TYPE_Q8_0, 160, [3000], 4096, 2), (O.TYPE_Q6_K, 160, [3000], 4096, 0),
                                         (O.TYPE_Q5_K, 160, [3000], 4096, 0), (O.TYPE_Q8_0, 140, [1024, 1024], 4096, 2),
                                         (O.TYPE_Q8_0, 160, [3000], 4096, 0), (O.TYPE_Q8_0, 140, [1024, 1024], 4096, 0)],
                         ids=["q8_0_fp16", "q6_K", "q5_K", "q8_0_group_fp16", "q8_0_int8", "q8_0_group_int8"])
def test_mul_mat_gemm_long_k(mx, be, t, M, Ns, K, q8):
    """Long products whose grid is small split K. On the fp16 GEMM they keep the 128 x 128 tile: ragged widths through
    the scalar reduce, a two-weight group of widths divisible by four through the vector one. On the int8 Q8_0 GEMM
    (32 stages of K): two splits of 64 x 64 tiles, ragged and grouped."""
    ws = [weights(t, n, K, 0x5EED1400 + n + t) for n in Ns]
    x = acts(0xAC701400 + M, M, K)
    W = [be.tensor(t, (K, n), w) for n, w in zip(Ns, ws)]
    X = be.tensor(mx.F32, (K, M), x)
    Y = [be.tensor(mx.F32, (n, M)) for n in Ns]
    with be.options(gemm_q8_0=q8):
        be.mul_mat_group(W, X, Y)
        be.sync()
    for n, w, yt in zip(Ns, ws, Y):
        check_product(t, w, x, yt.numpy().reshape(M, n), K, dq=None if t != O.TYPE_Q8_0 else q8 == 2)


def test_mul_mat_gemm_batched(mx, be):
    t, K, N, M = O.TYPE_Q8_0, 1024, 96, 40
    w = weights(t, N * 2, K, 0x5EED0B00)
    x = acts(0xAC700B00, M * 4, K).reshape(1, 4, M, K)
    W = be.tensor(t, (K, N, 2, 1), w)
    X = be.tensor(mx.F32, (K, M, 4, 1), x)
    Y = be.tensor(mx.F32, (N, M, 4, 1))
    be.mul_mat(W, X, Y)
    be.sync()
    y = Y.numpy()
    for i2 in range(4):
        wm = w[(i2 // 2) * N:(i2 // 2 + 1) * N]
        check_product(t, wm, x[0, i2], y[0, i2], K)


@pytest.mark.parametrize("t", [O.TYPE_Q4_K, O.TYPE_Q5_K, O.TYPE_Q6_K], ids=lambda t: NAMES[t])
@pytest.mark.parametrize("M,N,K", [(9, 100, 1024), (64, 256, 2048), (130, 333, 1536), (512, 1024, 3072),
                                   (100, 64, 6144)])
def test_mul_mat_gemm_kquant(mx, be, t, M, N, K):
    w = weights(t, N, K, 0x5EED0C00 + M + N + t)
    x = acts(0xAC700C00 + M, M, K)
    y = run_mul_mat(mx, be, t, w, x, K, N)
    check_product(t, w, x, y, K)


@pytest.mark.parametrize("t", QTYPES, ids=lambda t: NAMES[t])
def test_mul_mat_gemm_special_rows(mx, be, t):
    """Zero, constant, tied and subnormal-scale activation rows through the M > 8 path."""
    K, N = 1024, 160
    w = weights(t, N, K, 0x5EED0D00 + t)
    x = np.concatenate([special_rows(K), acts(0xAC700D00, 7, K)])
    y = run_mul_mat(mx, be, t, w, x, K, N)
    check_product(t, w, x, y, K)


@pytest.mark.parametrize("t", [O.TYPE_Q8_0, O.TYPE_Q5_K, O.TYPE_Q6_K], ids=lambda t: NAMES[t])
@pytest.mark.parametrize("K", [2048, 8192, 10240, 20480])
def test_mul_mat_gemm_activation_pass_widths(mx, be, t, K):
    """Rows of 2048 to 20480 elements through the activation pass before the fp16 GEMM: up to 16384 a row stays in
    registers while its largest |d q| is found, past that it is quantized twice; special and ordinary rows."""
    N = 64
    w = weights(t, N, K, 0x5EED1000 + t + K)
    x = np.concatenate([special_rows(K), acts(0xAC701000 + K, 7, K)])
    y = run_mul_mat(mx, be, t, w, x, K, N)
    check_product(t, w, x, y, K)


@pytest.mark.parametrize("t", [O.TYPE_Q4_K, O.TYPE_Q6_K], ids=lambda t: NAMES[t])
def test_mul_mat_gemm_kquant_batched(mx, be, t):
    """Broadcast batches: ne12 = 2 * ne02, each weight matrix serves two activation slices."""
    K, N, M = 1536, 96, 33
    w = weights(t, N * 2, K, 0x5EED0E00)
    x = acts(0xAC700E00, M * 4, K).reshape(1, 4, M, K)
    W = be.tensor(t, (K, N, 2, 1), w)
    X = be.tensor(mx.F32, (K, M, 4, 1), x)
    Y = be.tensor(mx.F32, (N, M, 4, 1))
    be.mul_mat(W, X, Y)
    be.sync()
    y = Y.numpy()
    for i2 in range(4):
        wm = w[(i2 // 2) * N:(i2 // 2 + 1) * N]
        check_product(t, wm, x[0, i2], y[0, i2], K)


@pytest.mark.parametrize("t", [O.TYPE_Q4_K, O.TYPE_Q6_K], ids=lambda t: NAMES[t])
def test_mul_mat_gemm_kquant_group(mx, be, t):
    """Two weights sharing src1 (gate / up): one Q8_K quantization, two GEMMs."""
    K, M = 2048, 70
    Ns = (192, 130)
    w = [weights(t, n, K, 0x5EED0F00 + n) for n in Ns]
    x = acts(0xAC700F00, M, K)
    W = [be.tensor(t, (K, n), wi) for n, wi in zip(Ns, w)]
    X = be.tensor(mx.F32, (K, M), x)
    Y = [be.tensor(mx.F32, (n, M)) for n in Ns]
    be.mul_mat_group(W, X, Y)
    be.sync()
    for n, wi, Yi in zip(Ns, w, Y):
        check_product(t, wi, x, Yi.numpy().reshape(M, n), K)


# ------------------------------------------------------------------------------------------- F16 / F32 weights
@pytest.mark.parametrize("t", FTYPES, ids=lambda t: NAMES[t])
def test_float_get_rows_bit_exact(mx, be, t):
    K, R = 1000, 40
    table = weights(t, R, K, 0x5EED1000 + t, std=1.0)
    ids = np.array([39, 0, 7, 7, 12], np.int32)
    T = be.tensor(t, (K, R), table)
    I = be.tensor(mx.I32, (len(ids),), ids)
    D = be.tensor(mx.F32, (K, len(ids)))
    be.get_rows(T, I, D)
    be.sync()
    assert bits_equal(D.numpy().reshape(len(ids), K), O.get_rows(t, table, K, ids))


@pytest.mark.parametrize("t", FTYPES, ids=lambda t: NAMES[t])
@pytest.mark.parametrize("M,K", [(1, 64), (1, 4096), (3, 1000), (8, 2048), (20, 1024)])
def test_float_mul_mat(mx, be, t, M, K):
    """ggml-cpu's F16 product rounds src1 to fp16 first; F32 takes it as it is. Missing that rounding would show as
    ~2e-4 of the row's largest output, ten times the bar held here."""
    N = 203
    w = weights(t, N, K, 0x5EED1100 + K + t)
    x = acts(0xAC701100 + M, M, K)
    y = run_mul_mat(mx, be, t, w, x, K, N)
    assert rel_err(y, O.mul_mat(t, w, x)) <= TIGHT
    assert rel_err(y, O.mul_mat(t, w, x, exact=True)) <= TIGHT


@pytest.mark.parametrize("t", FTYPES, ids=lambda t: NAMES[t])
def test_float_mul_mat_batched_group(mx, be, t):
    """Broadcast batches (ne12 = 2 ne02) and a two-weight group sharing src1."""
    K, N, M = 512, 72, 2
    w = weights(t, N * 2, K, 0x5EED1200 + t)
    x = acts(0xAC701200, M * 4, K).reshape(1, 4, M, K)
    W = be.tensor(t, (K, N, 2, 1), w)
    X = be.tensor(mx.F32, (K, M, 4, 1), x)
    Y = be.tensor(mx.F32, (N, M, 4, 1))
    be.mul_mat(W, X, Y)
    be.sync()
    y = Y.numpy()
    for i2 in range(4):
        wm = w[(i2 // 2) * N:(i2 // 2 + 1) * N]
        assert rel_err(y[0, i2], O.mul_mat(t, wm, x[0, i2])) <= TIGHT
    ws = [weights(t, n, K, 0x5EED1300 + n + t) for n in (96, 40)]
    Wg = [be.tensor(t, (K, n), wi) for n, wi in zip((96, 40), ws)]
    Xg = be.tensor(mx.F32, (K, 3), x.reshape(-1, K)[:3])
    Yg = [be.tensor(mx.F32, (n, 3)) for n in (96, 40)]
    be.mul_mat_group(Wg, Xg, Yg)
    be.sync()
    for n, wi, Yi in zip((96, 40), ws, Yg):
        assert rel_err(Yi.numpy().reshape(3, n), O.mul_mat(t, wi, x.reshape(-1, K)[:3])) <= TIGHT


# ------------------------------------------------------------------------------------------------------------ ARGMAX
def argmax_rows(n, R, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((R, n)).astype(np.float32)
    if R > 1:
        x[1, [5, n // 3, n - 1]] = 50.0                  # ties spread over threads and waves: the first
    if R > 2:
        x[2, :] = 0.25                                   # all equal
    if R > 3:
        x[3, 0] = np.nan                                 # NaN at index 0 wins by default
        x[3, 7] = 99.0
    if R > 4:
        x[4, [1, 100, n - 2]] = np.nan                   # NaNs elsewhere are passed over
        x[4, n // 2] = 77.0
    if R > 5:
        x[5, :] = -np.inf
    if R > 6:
        x[6, n - 1] = np.inf
    if R > 7:
        x[7, 4 * 37 + 2] = 30.0                          # one max inside a 16-byte group, and its tie in the next
        x[7, 4 * 38 + 1] = 30.0
    return x


@pytest.mark.parametrize("n,R", [(151936, 8), (3072, 11), (64, 3), (4, 1), (1000, 9)])
def test_argmax_matches_oracle(mx, be, n, R):
    x = argmax_rows(n, R, 0xA46 + n + R)
    X = be.tensor(mx.F32, (n, R), x)
    Y = be.tensor(mx.I32, (R,))
    be.argmax(X, Y)
    be.sync()
    assert np.array_equal(Y.numpy().reshape(R), O.argmax(x))


def test_argmax_rows_split_over_workgroups(mx, be):
    """A vocabulary-sized row is split over many workgroups: ties across the parts, a part that holds only NaNs and
    a NaN at index 0 still follow the first-of-equal rule."""
    n = 151936
    x = np.random.default_rng(0xA48).standard_normal((3, n)).astype(np.float32)
    x[0, [70001, 100, 151935]] = 50.0           # the first of three, in three parts
    x[1, 4096 * 5:4096 * 9] = np.nan           # whole parts of NaN
    x[1, [4096 * 9, 4096 * 30 + 3]] = 9.0      # tie in two parts
    x[2, 0] = np.nan                            # index 0 wins
    x[2, 77] = 1e30
    for R in (1, 3):
        X = be.tensor(mx.F32, (n, R), x[:R])
        Y = be.tensor(mx.I32, (R,))
        be.argmax(X, Y)
        be.sync()
        assert np.array_equal(Y.numpy().reshape(R), O.argmax(x[:R]))
    assert list(O.argmax(x)) == [100, 4096 * 9, 0]


def test_argmax_padded_rows(mx, be):
    """Rows whose length is not a multiple of four (the kernel's tail) inside 16-byte-aligned padded rows."""
    n, R, pitch = 1001, 6, 1008
    x = argmax_rows(n, R, 0xA47)
    xp = np.zeros((R, pitch), np.float32)
    xp[:, :n] = x
    xp[:, n:] = 1e30                                     # padding must never be read as a value
    X = mx.Tensor(be, mx.F32, (n, R), nb=(4, 4 * pitch, 4 * pitch * R, 4 * pitch * R))
    X.set(xp.reshape(-1)[: (R - 1) * pitch + n])
    Y = be.tensor(mx.I32, (R,))
    be.argmax(X, Y)
    be.sync()
    assert np.array_equal(Y.numpy().reshape(R), O.argmax(x))
