"""Every kernel the products' dispatcher can pick, reached in one process: by the shapes that pick it by default
(config 3's Q4_K prefill groups on the 128 x 128 eight-wave and 64 x 64 four-wave tiles) and by a backend's options
(mx_backend_set_option: the int8 Q8_0 GEMM's tiles and K splits, the fp16 GEMM on Q8_0, the VALU-scaled int8 K-quant
GEMM, each GEMM tile, forced K splits, the mat-vec's lanes per row, the MUL_MAT_ID experts kernel or grouped product
and its mat-vec threshold), each held to the oracle at the parity bars of test_gpu_parity.py. Also the graph rule that a graph recorded before the backend's scratch grew is
refused."""
import ctypes

import numpy as np
import pytest

import oracle as O
from helpers import rel_err
from test_gpu_parity import NAMES, TIGHT, acts, check_product, mmid_case, weights

pytestmark = pytest.mark.gpu


def run_products(mx, be, t, ws, Ns, x, K):
    """src0 = ws[i] ([Ns[i], K] quantized) times x ([M, K]) as one MUL_MAT (a single weight) or one group."""
    M = x.shape[0]
    W = [be.tensor(t, (K, n), w) for n, w in zip(Ns, ws)]
    X = be.tensor(mx.F32, (K, M), x)
    Y = [be.tensor(mx.F32, (n, M)) for n in Ns]
    if len(Ns) == 1:
        be.mul_mat(W[0], X, Y[0])
    else:
        be.mul_mat_group(W, X, Y)
    be.sync()
    return [y.numpy().reshape(M, n) for n, y in zip(Ns, Y)]


def case(t, M, Ns, K, seed):
    ws = [weights(t, n, K, seed + 7 * i) for i, n in enumerate(Ns)]
    x = acts(seed + 1, M, K)
    refs = [O.mul_mat_par(t, w, x) for w in ws]
    return ws, x, refs


# --------------------------------------------------------------------------------------- Q4_K prefill (config 3)
# (M, widths, K): config 3's q/k/v group (128 workgroups of 128 x 128, so 512 of 64 x 64 by default), its gate/up
# group (384 of 128 x 128 by default), attn_o (64 of 128 x 128, so 256 of 64 x 64) and a ragged product (192 of
# 128 x 128, so 64 x 64 tiles with partial rows and columns).
Q4K_SHAPES = {"qkv": (512, [2048, 1024, 1024], 2048), "gate_up": (512, [6144, 6144], 2048),
              "attn_o": (512, [2048], 2048), "ragged": (300, [8100], 256)}


@pytest.mark.parametrize("shape", list(Q4K_SHAPES))
def test_q4k_gemm_config3_every_tile(mx, be, shape):
    M, Ns, K = Q4K_SHAPES[shape]
    t = O.TYPE_Q4_K
    ws, x, refs = case(t, M, Ns, K, 0x5EED3000 + len(Ns) * 100 + M)
    for tile in [(0, 0), (128, 128), (128, 64), (64, 128), (64, 64)]:
        with be.options(tile_m=tile[0], tile_n=tile[1]):
            ys = run_products(mx, be, t, ws, Ns, x, K)
        for w, y, r in zip(ws, ys, refs):
            assert rel_err(y, r) <= TIGHT, f"tile {tile}"


# --------------------------------------------------------------------------------------- Q8_0 on int8 MFMA
# config 4's shapes: the q/k/v group at M = 512, down (K = 6144), a short 28-row block, and a ragged product
I8_SHAPES = {"qkv": (512, [2048, 1024, 1024], 2048), "down": (512, [2048], 6144), "short": (28, [2048], 2048),
             "ragged": (130, [333], 1024)}


@pytest.mark.parametrize("shape", list(I8_SHAPES))
def test_q8_0_int8_gemm_every_tile_and_split(mx, be, shape):
    M, Ns, K = I8_SHAPES[shape]
    t = O.TYPE_Q8_0
    ws, x, refs = case(t, M, Ns, K, 0x5EED3100 + M + K)
    for tile in [(0, 0), (64, 64), (64, 128), (128, 128)]:
        for split in (0, 1, 3, 64):  # 64: more than the 128-wide stages of K, so one split per stage
            with be.options(gemm_q8_0=1, tile_m=tile[0], tile_n=tile[1], split=split):
                ys = run_products(mx, be, t, ws, Ns, x, K)
            for w, y, r in zip(ws, ys, refs):
                check_product(t, w, x, y, K, int8=True, y_ref=r)


# --------------------------------------------------------------------------------------- VALU-scaled int8 K-quants
@pytest.mark.parametrize("t", [O.TYPE_Q4_K, O.TYPE_Q6_K], ids=lambda t: NAMES[t])
@pytest.mark.parametrize("M,Ns,K", [(512, [2048], 2048), (512, [2048], 6144), (130, [333], 1536),
                                    (70, [192, 130], 2048)], ids=["m512", "down", "ragged", "group"])
def test_kquant_int8_gemm(mx, be, t, M, Ns, K):
    ws, x, refs = case(t, M, Ns, K, 0x5EED3200 + M + K + t)
    with be.options(gemm_kquant=1):
        ys = run_products(mx, be, t, ws, Ns, x, K)
    for w, y, r in zip(ws, ys, refs):
        check_product(t, w, x, y, K, int8=True, y_ref=r)


# --------------------------------------------------------------------------------------- fp16 dequantizing GEMM
FP16_Q8 = {"gemm_q8_0": 2}  # Q8_0 products on the fp16 GEMM (the int8 one is picked where K % 128 == 0)

@pytest.mark.parametrize("t", [O.TYPE_Q8_0, O.TYPE_Q5_K, O.TYPE_Q6_K], ids=lambda t: NAMES[t])
def test_dq_gemm_every_tile_and_split(mx, be, t):
    M, N, K = 300, 1000, 2048
    ws, x, refs = case(t, M, [N], K, 0x5EED3300 + t)
    for tile in [(64, 64), (128, 64), (128, 128), (64, 128)]:  # 64 x 128: the direct-B tile of four 64 x 32 waves
        for split in (1, 3):
            with be.options(tile_m=tile[0], tile_n=tile[1], split=split, **FP16_Q8):
                y = run_products(mx, be, t, ws, [N], x, K)[0]
            check_product(t, ws[0], x, y, K, y_ref=refs[0], dq=True)


@pytest.mark.parametrize("t", [O.TYPE_Q8_0, O.TYPE_Q5_K, O.TYPE_Q6_K], ids=lambda t: NAMES[t])
@pytest.mark.parametrize("M", [28, 9, 40])
def test_dq_gemm_short_blocks(mx, be, t, M):
    """Blocks of at most 32 rows (a prompt's last, short block: 28 rows of the 1564-row ASR prompt) take the 32 x 128
    tile of the direct-B types with K split so that about 256 workgroups stream the weights; it is held to the same
    model of the fp16 GEMM at its picked split and at forced ones (one split; three; a ragged N), and at 40 rows (two
    row tiles) when forced."""
    for N, K in ((1000, 2048), (2048, 6144), (333, 1024)):
        ws, x, refs = case(t, M, [N], K, 0x5EED3500 + M + N)
        for split in ((0, 1, 3) if M <= 32 else (0,)):
            with be.options(tile_m=32, tile_n=128, split=split, **FP16_Q8):
                y = run_products(mx, be, t, ws, [N], x, K)[0]
            check_product(t, ws[0], x, y, K, y_ref=refs[0], dq=True)
        if M <= 32:  # picked without the tile options
            with be.options(**FP16_Q8):
                y = run_products(mx, be, t, ws, [N], x, K)[0]
            check_product(t, ws[0], x, y, K, y_ref=refs[0], dq=True)


def test_dq_gemm_tiny_rows(mx, be):
    """Q8_K rows whose largest |d q| is ~1e-35 (below 2^-112): the row's power-of-two scale stays a normal float,
    so the outputs keep their size instead of becoming zero."""
    t, M, N, K = O.TYPE_Q6_K, 12, 160, 1024
    ws = [weights(t, N, K, 0x5EED3400)]
    x = acts(0xAC703400, M, K)
    x[:4] *= np.float32(1e-35)
    y = run_products(mx, be, t, ws, [N], x, K)[0]
    check_product(t, ws[0], x, y, K)
    assert np.abs(y[:4]).max() > 0


# --------------------------------------------------------------------------------------- mat-vec lanes per row
@pytest.mark.parametrize("t,K", [(O.TYPE_Q8_0, 1024), (O.TYPE_Q8_0, 3072), (O.TYPE_Q4_K, 2048), (O.TYPE_Q4_K, 2816),
                                 (O.TYPE_Q4_K, 6144), (O.TYPE_Q6_K, 3072), (O.TYPE_Q5_K, 1536)], ids=lambda v: str(v))
def test_matvec_every_lanes_per_row(mx, be, t, K):
    N = 333
    for M in (1, 3):
        ws, x, refs = case(t, M, [N], K, 0x5EED3500 + t + K + M)
        for lpr in (16, 32, 64):
            with be.options(matvec_lpr=lpr):
                y = run_products(mx, be, t, ws, [N], x, K)[0]
            assert rel_err(y, refs[0]) <= TIGHT, f"lanes per row {lpr}"


# --------------------------------------------------------------------------------------- MUL_MAT_ID paths
@pytest.mark.parametrize("t", [O.TYPE_Q8_0, O.TYPE_Q4_K, O.TYPE_Q6_K], ids=lambda t: NAMES[t])
def test_mmid_every_path(mx, be, t):
    """The experts kernel where the grouped product would run (Q4_K: the int8 grouped product; Q8_0, Q6_K: the fp16
    GEMM over each expert's chunks), in several passes per expert (40 tokens) and in its one-pass form (16 tokens);
    the grouped product forced at a small batch; the bucketed path for a single token (mat-vec threshold 0); the
    mat-vec path for 64 pairs (threshold 64); the Q4_K grouped product's chunk forms where the other one would be
    picked (the fp16 GEMM keeps its one chunk size)."""
    with be.options(mmid_kernel=1):
        y, ref = mmid_case(mx, be, t, E=16, K=1024, N=200, n_ids=4, T=40, bcast=False, seed=0x5EED3600 + t)
        ref.check(y)
    with be.options(mmid_kernel=2):
        y, ref = mmid_case(mx, be, t, E=16, K=1024, N=200, n_ids=4, T=16, bcast=True, seed=0x5EED3630 + t)
        ref.check(y)
    with be.options(mmid_kernel=1):
        y, ref = mmid_case(mx, be, t, E=64, K=2048, N=192, n_ids=4, T=16, bcast=True, seed=0x5EED3640 + t)
        ref.check(y)
    for chunk in (16, 32):  # the grouped product's one-tile form at 40 tokens, its two-tile form at 16
        with be.options(mmid_chunk=chunk):
            y, ref = mmid_case(mx, be, t, E=16, K=1024, N=200, n_ids=4, T=40 if chunk == 16 else 16, bcast=False,
                               seed=0x5EED3650 + t + chunk)
            ref.check(y, f"chunks of {chunk}")
    with be.options(mmid_matvec_pairs=0):
        y, ref = mmid_case(mx, be, t, E=16, K=1024, N=200, n_ids=4, T=1, bcast=True, seed=0x5EED3610 + t)
        ref.check(y)
    with be.options(mmid_matvec_pairs=64):
        y, ref = mmid_case(mx, be, t, E=16, K=1024, N=200, n_ids=4, T=16, bcast=False, seed=0x5EED3620 + t)
        ref.check(y)


@pytest.mark.parametrize("t", [O.TYPE_Q8_0, O.TYPE_Q5_K, O.TYPE_Q6_K], ids=lambda t: NAMES[t])
@pytest.mark.parametrize("tile", [(32, 128), (32, 64), (64, 64)], ids=lambda v: f"{v[0]}x{v[1]}")
def test_mmid_dq_every_tile(mx, be, t, tile):
    """The fp16 GEMM over expert chunks on each of its tiles (a chunk per row tile: 32 or 64 of an expert's pairs),
    with experts of 0, 1, 31, 32, 33, 64, 65 and 100 pairs (full, ragged and several chunks), N not a multiple of the
    column tile, b broadcast over the slots and per slot."""
    counts = [1, 31, 0, 32, 33, 64, 65, 100]
    ids = np.concatenate([np.full(c, e, np.int32) for e, c in enumerate(counts)])
    np.random.default_rng(9).shuffle(ids)
    with be.options(mmid_kernel=2, tile_m=tile[0], tile_n=tile[1]):
        y, ref = mmid_case(mx, be, t, E=len(counts), K=1024, N=200, n_ids=1, T=len(ids), bcast=True,
                           seed=0x5EED3700 + t, ids=ids.reshape(-1, 1))
        ref.check(y, "b broadcast")
        y, ref = mmid_case(mx, be, t, E=16, K=1536, N=136, n_ids=4, T=40, bcast=False, seed=0x5EED3710 + t)
        ref.check(y, "b per slot")


# --------------------------------------------------------------------------------------- refusals
def test_options_refused(mx, be):
    for name, bad in [("gemm_q8_0", 3), ("tile_m", 96), ("matvec_lpr", 8), ("split", -1), ("mmid_matvec_pairs", -1),
                      ("mmid_kernel", 3), ("mmid_chunk", 8)]:
        with pytest.raises(mx.MxError) as e:
            be.set_option(name, bad)
        assert e.value.code == mx.INVALID
    with pytest.raises(mx.MxError) as e:
        mx.check(mx.lib().mx_backend_set_option(be.h, 99, 0))
    assert e.value.code == mx.INVALID
    t, M, N, K = O.TYPE_Q8_0, 16, 64, 1056  # K not a multiple of 128: the int8 Q8_0 GEMM cannot take it
    ws = [weights(t, N, K, 0x5EED3700)]
    x = acts(0xAC703700, M, K)
    with be.options(gemm_q8_0=1):
        with pytest.raises(mx.MxError) as e:
            run_products(mx, be, t, ws, [N], x, K)
        assert e.value.code == mx.UNSUPPORTED
    t, K = O.TYPE_Q4_K, 1024  # a 32 x 128 tile the Q4_K GEMM lacks
    ws = [weights(t, N, K, 0x5EED3701)]
    x = acts(0xAC703701, M, K)
    with be.options(tile_m=32, tile_n=128):
        with pytest.raises(mx.MxError) as e:
            run_products(mx, be, t, ws, [N], x, K)
        assert e.value.code == mx.FAILED
    assert be.get_option("tile_m") == 0 and be.get_option("gemm_q8_0") == 0


# --------------------------------------------------------------------------------------- graphs and scratch
def test_graph_refused_after_scratch_grows(mx):
    """A graph holds the scratch address it was recorded with. Once a larger op reallocates the scratch, launching
    that graph fails with MX_FAILED (it would read freed memory); a graph recorded again replays correctly. A graph
    launches only on the backend that recorded it."""
    be = mx.Backend(0)
    other = mx.Backend(0)
    try:
        t, K = O.TYPE_Q8_0, 1024
        w = weights(t, 256, K, 0x5EED3800)
        x = acts(0xAC703800, 16, K)
        W = be.tensor(t, (K, 256), w)
        X = be.tensor(mx.F32, (K, 16), x)
        Y = be.tensor(mx.F32, (256, 16))
        be.mul_mat(W, X, Y)
        be.sync()
        be.graph_begin()
        be.mul_mat(W, X, Y)
        g = be.graph_end()
        be.graph_launch(g)
        be.sync()
        with pytest.raises(mx.MxError) as e:
            other.graph_launch(g)
        assert e.value.code == mx.INVALID
        # a product whose activations need far more scratch than the first
        K2, M2 = 4096, 512
        W2 = be.tensor(t, (K2, 64), weights(t, 64, K2, 0x5EED3801))
        X2 = be.tensor(mx.F32, (K2, M2), acts(0xAC703801, M2, K2))
        Y2 = be.tensor(mx.F32, (64, M2))
        be.mul_mat(W2, X2, Y2)
        be.sync()
        with pytest.raises(mx.MxError) as e:
            be.graph_launch(g)
        assert e.value.code == mx.FAILED
        be.graph_free(g)
        Y.set(np.zeros((16, 256), np.float32))
        be.graph_begin()
        be.mul_mat(W, X, Y)
        g = be.graph_end()
        be.graph_launch(g)
        be.sync()
        check_product(t, w, x, Y.numpy().reshape(16, 256), K)
        be.graph_free(g)
    finally:
        other.close()
        be.close()


# --------------------------------------------------------------------------------------- peak micro-benchmarks
def test_peak_entry_points(mx, be):
    """mx_peak_read / mx_peak_mfma run (small sizes) and refuse what they cannot take."""
    buf = be.tensor(mx.F32, (1 << 20,))
    be.peak_read(buf, 64, 4)
    be.peak_read(buf, 64, 16, nontemporal=True)
    be.peak_mfma(0, 8, 10)
    be.peak_mfma(1, 8, 10)
    be.sync()
    L = mx.lib()
    for rc in (L.mx_peak_read(be.h, ctypes.c_void_p(buf.base), 100, 64, 4, 0),        # not whole 16-byte chunks
               L.mx_peak_read(be.h, ctypes.c_void_p(buf.base + 4), 4096, 64, 4, 0),   # misaligned
               L.mx_peak_read(be.h, ctypes.c_void_p(buf.base), 4096, 64, 3, 0),       # loads in flight
               L.mx_peak_read(be.h, ctypes.c_void_p(buf.base), 4096, 0, 4, 0),        # no workgroups
               L.mx_peak_mfma(be.h, 2, 8, 10), L.mx_peak_mfma(be.h, 0, 8, 0)):
        assert rc == mx.INVALID
    buf.free()
