"""A seeded sweep of product shapes across the dispatcher's boundaries, every weight type, through the C ABI on
device 0: MUL_MAT at row counts either side of the mat-vec / GEMM switch (8 | 9) and the short-block tile (32 | 33),
K with and without the GEMMs' multiples (Q8_0 K % 64 for the fp16 GEMM, K % 128 for the int8 one), ragged N; MUL_MAT_ID with pair counts either side of the
mat-vec launch (16) and of the fp16 GEMM's per-expert thresholds (one pair per expert for Q8_0, three for the
K-quants), b broadcast and per slot. Each case is held to its path's bar (test_gpu_parity.py): the integer paths to
2e-5 of the oracle, the fp16 dequantizing GEMM to 1e-3 of it and to 2e-5 of a model of its roundings. A product of
fewer than 32 outputs per row (N = 1 .. 31) is measured against its largest output over all rows instead of each
row's own: with one or a few outputs a row's maximum can sit near zero, and the row-relative error becomes the
relative error of single values. The draws are fixed by the seed, so a failure names its case."""
import numpy as np
import pytest

import oracle as O
from helpers import dq_model
from test_gpu_parity import NAMES, QTYPES, TIGHT, TOL, acts, check_product, mmid_case, uses_dq, weights

pytestmark = pytest.mark.gpu

M_SET = [1, 2, 5, 8, 9, 16, 28, 32, 33, 64, 130, 300]
N_SET = [1, 7, 31, 100, 129, 333, 1000]
K_SET = {O.TYPE_Q8_0: [32, 96, 256, 1056, 2048, 4096], O.TYPE_Q4_K: [256, 512, 1280, 2048, 3072],
         O.TYPE_Q5_K: [256, 768, 1536, 2048], O.TYPE_Q6_K: [256, 1024, 1536, 4096]}


def check_narrow(t, w, x, y, K):
    """check_product's bars, each error over the product's largest |output| (rows of fewer than 32 outputs)."""
    y_ref = O.mul_mat(t, w, x)
    scale = max(float(np.abs(y_ref).max()), 1e-30)
    err = lambda a, b: float(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64)).max()) / scale
    if uses_dq(t, x.shape[0], K):
        assert err(y, y_ref) <= TOL
        assert err(y, dq_model(O, t, w, x, K)) <= TIGHT
    else:
        assert err(y, y_ref) <= TIGHT


def draws(seed, n, *sets):
    rng = np.random.default_rng(seed)
    return [tuple(int(s[rng.integers(len(s))]) for s in sets) for _ in range(n)]


@pytest.mark.parametrize("t", QTYPES, ids=lambda t: NAMES[t])
def test_mul_mat_shape_sweep(mx, be, t):
    for i, (M, N, K) in enumerate(draws(0x5EED7000 + t, 14, M_SET, N_SET, K_SET[t])):
        w = weights(t, N, K, 0x5EED7100 + 31 * i + t)
        x = acts(0xAC707100 + 31 * i + t, M, K)
        W, X, Y = be.tensor(t, (K, N), w), be.tensor(mx.F32, (K, M), x), be.tensor(mx.F32, (N, M))
        be.mul_mat(W, X, Y)
        be.sync()
        y = Y.numpy().reshape(M, N)
        try:
            (check_product if N >= 32 else check_narrow)(t, w, x, y, K)
        except AssertionError as e:
            raise AssertionError(f"draw {i}: M {M} N {N} K {K}") from e


E_SET = [4, 8, 16, 64]
NIDS_SET = [1, 2, 4, 8]
T_SET = [1, 3, 9, 17, 40, 100]
MMID_N_SET = [32, 100, 136]


@pytest.mark.parametrize("t", QTYPES, ids=lambda t: NAMES[t])
def test_mul_mat_id_shape_sweep(mx, be, t):
    ks = [k for k in K_SET[t] if k >= 256]
    for i, (E, n_ids, T, N, K, b) in enumerate(draws(0x5EED7200 + t, 10, E_SET, NIDS_SET, T_SET, MMID_N_SET, ks,
                                                     [0, 1])):
        n_ids = min(n_ids, E)
        y, ref = mmid_case(mx, be, t, E=E, K=K, N=N, n_ids=n_ids, T=T, bcast=bool(b), seed=0x5EED7300 + 31 * i + t)
        ref.check(y, f"draw {i}: E {E} n_ids {n_ids} T {T} N {N} K {K} b {'broadcast' if b else 'per slot'}")


@pytest.mark.parametrize("seed", range(3))
def test_int8_q8_0_gemm_group_sweep(mx, be, seed):
    """The int8 Q8_0 GEMM (the default for Q8_0 at M > 8, K % 128 == 0) over seeded groups: one to four weights of
    ragged widths sharing the activations, M from 9 to 600, K from one 128-wide stage to 48, at the picked tile and
    split and at a forced split; every output to TIGHT of the oracle's exact block sums."""
    rng = np.random.default_rng(0x5EED7400 + seed)
    t = O.TYPE_Q8_0
    for i in range(4):
        M = int(rng.choice([9, 17, 33, 64, 100, 200, 600]))
        K = 128 * int(rng.choice([1, 2, 5, 8, 16, 48]))
        Ns = [int(rng.integers(1, 700)) for _ in range(int(rng.integers(1, 5)))]
        split = int(rng.choice([0, 0, 2, 3, 7]))
        ws = [weights(t, n, K, 0x5EED7500 + 97 * seed + 13 * i + j) for j, n in enumerate(Ns)]
        x = acts(0xAC707500 + 97 * seed + i, M, K)
        W = [be.tensor(t, (K, n), w) for n, w in zip(Ns, ws)]
        X = be.tensor(mx.F32, (K, M), x)
        Y = [be.tensor(mx.F32, (n, M)) for n in Ns]
        with be.options(split=split):
            be.mul_mat_group(W, X, Y)
            be.sync()
        for n, w, yt in zip(Ns, ws, Y):
            y = yt.numpy().reshape(M, n)
            try:
                (check_product if n >= 32 else check_narrow)(t, w, x, y, K)
            except AssertionError as e:
                raise AssertionError(f"draw {i}: M {M} widths {Ns} K {K} split {split}") from e
