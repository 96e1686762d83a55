"""MUL_MAT_ID through the entry point that allocates nothing (mx_mul_mat_id_noalloc: its scratch a static device
array per GPU) against mx_mul_mat_id on the same inputs: the same kernels, so the same bits, on two calls in a row
(the second smaller, so it runs on what the first left in the shared array), for Q4_K experts (the grouped MFMA
kernel) and Q8_0 experts (the generic kernel); both held to the oracle. A call needing more than the array holds is
refused before anything runs."""
import numpy as np
import pytest

import oracle as O
from helpers import bits_equal, rel_err

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
    for T, n_ids, N in [(40, 4, 200), (9, 2, 72)]:  # the second call smaller than the first
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
        assert rel_err(yn, O.mul_mat_id(t, w, x, ids)) <= TIGHT


def test_mul_mat_id_noalloc_refuses_beyond_its_scratch(mx, be):
    t, E, K, N, n_ids, T = O.TYPE_Q8_0, 4, 4096, 32, 1, 4200
    need = mx.lib().mx_mul_mat_id_noalloc_bytes(
        be.tensor(t, (K, N, E)).ref(), be.tensor(mx.F32, (K, n_ids, 1)).ref(), be.tensor(mx.I32, (n_ids, T)).ref())
    assert need > mx.NOALLOC_SCRATCH_BYTES
    Wt = be.tensor(t, (K, N, E))
    Xt = be.tensor(mx.F32, (K, n_ids, T))
    It = be.tensor(mx.I32, (n_ids, T), np.zeros((T, n_ids), np.int32))
    Y = be.tensor(mx.F32, (N, n_ids, T))
    with pytest.raises(mx.MxError) as e:
        be.mul_mat_id_noalloc(Wt, Xt, It, Y)
    assert e.value.code == mx.UNSUPPORTED
