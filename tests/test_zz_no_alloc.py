"""MUL_MAT_ID through the entry point that allocates nothing (mx_mul_mat_id_noalloc: its scratch a static device
array per GPU) against mx_mul_mat_id on the same inputs: the same kernels, so the same bits, on two calls in a row
(the second smaller, so it runs on what the first left in the shared array), for Q4_K experts (the grouped int8
MFMA kernel) and Q8_0 experts (the fp16 dequantizing GEMM over each expert's chunks), and for 16 or fewer pairs (the
mat-vec launch); both held to the oracle at their paths' bars. Recorded into a graph -- what a caller that cannot allocate does -- and replayed with new inputs between the
replays, each replay matches the allocating entry point. A call needing more than the array holds is refused before
anything runs, and inputs MUL_MAT_ID does not take never size as fitting."""
import numpy as np
import pytest

import oracle as O
from helpers import bits_equal, rel_err
from test_gpu_parity import MmidRef, mmid_uses_dq

pytestmark = pytest.mark.gpu

TIGHT = 2e-5


def case(mx, be, t, E, K, N, n_ids, T, seed):
    w = O.quantize_chunk(t, O.fill_normal(seed, E * N, K, 0.0, 0.02)).reshape(E, N, -1)
    x = O.fill_normal(seed + 1, T * n_ids, K).reshape(T, n_ids, K)
    rng = np.random.default_rng(seed)
    ids = np.argsort(-rng.standard_normal((T, E)), axis=1)[:, :n_ids].astype(np.int32)
    Wt = be.tensor(t, (K, N, E), w.reshape(E * N, -1))
    Xt = be.tensor(mx.F32, (K, n_ids, T), x)
    It = be.tensor(mx.I32, (n_ids, T), ids)
    return w, x, ids, Wt, Xt, It


@pytest.mark.parametrize("t", [O.TYPE_Q4_K, O.TYPE_Q8_0], ids=["q4_K", "q8_0"])
def test_mul_mat_id_noalloc_matches_the_allocating_entry_point(mx, be, t):
    # the second call smaller than the first; the third of 3 x 4 = 12 pairs, on the mat-vec launch
    for T, n_ids, N in [(40, 4, 200), (9, 2, 72), (3, 4, 64)]:
        E, K = 16, 1024
        w, x, ids, Wt, Xt, It = case(mx, be, t, E, K, N, n_ids, T, 0x5EED6000 + T + t)
        Ya = be.tensor(mx.F32, (N, n_ids, T))
        Yn = be.tensor(mx.F32, (N, n_ids, T))
        be.mul_mat_id(Wt, Xt, It, Ya)
        be.mul_mat_id_noalloc(Wt, Xt, It, Yn)
        be.sync()
        ya = Ya.numpy().reshape(T, n_ids, N)
        yn = Yn.numpy().reshape(T, n_ids, N)
        assert bits_equal(yn, ya), f"T = {T}"
        MmidRef(t, w, x, ids, K, mmid_uses_dq(t, K, n_ids * T, E)).check(yn, f"T = {T}")


@pytest.mark.parametrize("pairs", [(24, 4), (4, 4)], ids=["grouped", "matvec"])
def test_mul_mat_id_noalloc_recorded_and_replayed(mx, be, pairs):
    """The call recorded into a graph and replayed three times, the inputs rewritten and the allocating entry point
    run eagerly between the replays (the array keeps the last call's contents): every replay matches it bit for bit
    and the oracle."""
    t, E, K, N = O.TYPE_Q4_K, 16, 1024, 128
    T, n_ids = pairs
    w, x, ids, Wt, Xt, It = case(mx, be, t, E, K, N, n_ids, T, 0x5EED6100 + T)
    Ya, Yn = be.tensor(mx.F32, (N, n_ids, T)), be.tensor(mx.F32, (N, n_ids, T))
    be.sync()
    be.graph_begin()
    be.mul_mat_id_noalloc(Wt, Xt, It, Yn)
    g = be.graph_end()
    try:
        rng = np.random.default_rng(0x5EED6200 + T)
        for r in range(3):
            x = O.fill_normal(0x5EED6300 + 16 * r + T, T * n_ids, K).reshape(T, n_ids, K)
            ids = np.argsort(-rng.standard_normal((T, E)), axis=1)[:, :n_ids].astype(np.int32)
            Xt.set(x)
            It.set(ids)
            be.graph_launch(g)
            be.sync()
            yn = Yn.numpy().reshape(T, n_ids, N).copy()
            be.mul_mat_id(Wt, Xt, It, Ya)
            be.sync()
            assert bits_equal(yn, Ya.numpy().reshape(T, n_ids, N)), f"replay {r}"
            assert rel_err(yn, O.mul_mat_id(t, w, x, ids)) <= TIGHT
    finally:
        be.graph_free(g)


def test_mul_mat_id_noalloc_refuses_beyond_its_scratch(mx, be):
    t, E, K, N, n_ids, T = O.TYPE_Q8_0, 4, 4096, 32, 1, 4200
    bytes_ = mx.lib().mx_mul_mat_id_noalloc_bytes
    need = bytes_(be.tensor(t, (K, N, E)).ref(), be.tensor(mx.F32, (K, n_ids, T)).ref(),
                  be.tensor(mx.I32, (n_ids, T)).ref())
    assert mx.NOALLOC_SCRATCH_BYTES < need < 1 << 40
    # inputs it cannot size: F32 experts, rows of another K, ids of another token count
    size_max = (1 << 64) - 1
    assert bytes_(be.tensor(mx.F32, (K, N, E)).ref(), be.tensor(mx.F32, (K, 1, 8)).ref(),
                  be.tensor(mx.I32, (n_ids, 8)).ref()) == size_max
    assert bytes_(be.tensor(t, (K, N, E)).ref(), be.tensor(mx.F32, (K // 2, 1, 8)).ref(),
                  be.tensor(mx.I32, (n_ids, 8)).ref()) == size_max
    assert bytes_(be.tensor(t, (K, N, E)).ref(), be.tensor(mx.F32, (K, 1, 8)).ref(),
                  be.tensor(mx.I32, (n_ids, 9)).ref()) == size_max
    Wt = be.tensor(t, (K, N, E))
    Xt = be.tensor(mx.F32, (K, n_ids, T))
    It = be.tensor(mx.I32, (n_ids, T), np.zeros((T, n_ids), np.int32))
    Y = be.tensor(mx.F32, (N, n_ids, T))
    with pytest.raises(mx.MxError) as e:
        be.mul_mat_id_noalloc(Wt, Xt, It, Y)
    assert e.value.code == mx.UNSUPPORTED
