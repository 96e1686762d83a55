"""Pins of the oracle's restatement of the decoder layer's other ops (RMS_NORM, ADD / MUL, SWIGLU, ROPE NEOX,
SET_ROWS, FLASH_ATTN_EXT), each against numpy arithmetic written here from the ops' definitions, closed forms and
properties; mutation checks show that a plausible mistake (a wrong pair layout, a dropped scale, a wrong KV head)
fails them."""
import numpy as np
import pytest

import oracle as O


def test_rms_norm_against_float64():
    x = np.concatenate([O.fill_normal(1, 5, 1024), O.fill_normal(2, 2, 128).repeat(8, axis=1)])
    y = O.rms_norm(x, 1e-6)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd * xd).mean(axis=1, keepdims=True) + 1e-6)
    assert np.abs(y - ref).max() <= 4e-7 * np.abs(ref).max()
    # closed form: a constant row c gives c / sqrt(c^2 + eps)
    c = np.full((1, 256), 3.0, np.float32)
    assert np.allclose(O.rms_norm(c, 0.0), 1.0, atol=0, rtol=1e-7)


def test_rms_norm_follows_the_float_mean():
    """The mean is rounded to float before eps is added (ggml's `const float mean = sum/ne00`): a row whose exact mean
    is not a float shows it against the double-throughout form, bit for bit."""
    x = (np.arange(1, 129, dtype=np.float32) * np.float32(0.1)).reshape(1, -1)
    sq = (x * x).astype(np.float64)                    # squares rounded to float, summed exactly
    mean = np.float32(sq.sum() / x.shape[1])
    scale = np.float32(1.0) / np.sqrt(mean + np.float32(1e-6), dtype=np.float32)
    assert np.array_equal(O.rms_norm(x, 1e-6), (x * scale).astype(np.float32))


def test_binary_broadcast_bit_exact():
    a = O.fill_normal(3, 6, 64)
    b1 = O.fill_normal(4, 1, 64)
    b3 = O.fill_normal(5, 3, 64)
    assert np.array_equal(O.binary("add", a, b1), a + b1)
    assert np.array_equal(O.binary("mul", a, b1), a * b1)
    assert np.array_equal(O.binary("mul", a, b3), a * np.tile(b3, (2, 1)))


def test_swiglu_against_float64():
    a = O.fill_normal(6, 4, 3072) * np.float32(4)
    b = O.fill_normal(7, 4, 3072)
    ad = a.astype(np.float64)
    ref = ad / (1 + np.exp(-ad)) * b
    assert np.abs(O.swiglu(a, b) - ref).max() <= 1e-6 * np.abs(ref).max()


def rope_numpy(x, pos, n_dims, base):
    """NEOX rotation written from ggml_rope_cache_init: float32 chain of angles, pairs (k, k + n_dims/2)."""
    rows, n_head, ne0 = x.shape
    half = n_dims // 2
    ts = np.float32(np.power(np.float32(base), np.float32(-2.0) / np.float32(n_dims), dtype=np.float32))
    y = x.astype(np.float64).copy()
    for r in range(rows):
        theta = np.float32(pos[r])
        ang = np.zeros(half, np.float32)
        for k in range(half):
            ang[k] = theta
            theta = np.float32(theta * ts)
        c, s = np.cos(ang.astype(np.float64)), np.sin(ang.astype(np.float64))
        x0, x1 = x[r, :, :half].astype(np.float64), x[r, :, half:n_dims].astype(np.float64)
        y[r, :, :half] = x0 * c - x1 * s
        y[r, :, half:n_dims] = x0 * s + x1 * c
    return y


def test_rope_neox_against_numpy():
    x = O.fill_normal(8, 5 * 16, 128).reshape(5, 16, 128)
    pos = np.array([0, 1, 37, 1000, 4095], np.int32)
    y = O.rope_neox(x, pos, 128, 1e6)
    ref = rope_numpy(x, pos, 128, 1e6)
    assert np.abs(y - ref).max() <= 2e-6
    assert np.array_equal(y[0], x[0])  # position 0 turns nothing
    # every pair keeps its length
    n0 = np.hypot(x[..., :64].astype(np.float64), x[..., 64:].astype(np.float64))
    n1 = np.hypot(y[..., :64].astype(np.float64), y[..., 64:].astype(np.float64))
    assert np.abs(n0 - n1).max() <= 1e-5
    # mutation: adjacent pairs (the non-NEOX layout) are a different rotation
    xs = x.reshape(5, 16, 64, 2).transpose(0, 1, 3, 2).reshape(5, 16, 128)
    assert np.abs(O.rope_neox(xs, pos, 128, 1e6) - ref).max() > 1e-2


def test_set_rows_f16():
    cache = np.zeros((8, 32), np.uint16)
    src = O.fill_normal(9, 3, 32) * np.float32(100)
    out = O.set_rows_f16(cache, src, np.array([5, 0, 7], np.int32))
    assert np.array_equal(out[[5, 0, 7]], src.astype(np.float16).view(np.uint16))
    assert not out[[1, 2, 3, 4, 6]].any()
    with pytest.raises(ValueError):
        O.set_rows_f16(cache, src, np.array([5, 8, 0], np.int32))


def attn_numpy(q, k, v, mask, scale):
    """Softmax attention in float64 over fp16-rounded q, written from the definition (GQA: head h reads kv head
    h // (n_head / n_kv_head)); output [n_q, n_head, D]."""
    n_head, n_q, D = q.shape
    n_kv_head = k.shape[0]
    qh = q.astype(np.float16).astype(np.float64)
    kf = k.view(np.float16).astype(np.float64)
    vf = v.view(np.float16).astype(np.float64)
    out = np.zeros((n_q, n_head, D))
    for h in range(n_head):
        hk = h // (n_head // n_kv_head)
        s = qh[h] @ kf[hk].T * scale
        if mask is not None:
            s = s + mask.view(np.float16).astype(np.float64)[:n_q, :k.shape[1]]
        m = s.max(axis=1, keepdims=True)
        p = np.exp(s - m)
        p[np.isinf(s)] = 0
        out[:, h] = (p @ vf[hk]) / p.sum(axis=1, keepdims=True)
    return out


def fa_case(seed, n_head, n_kv_head, n_q, n_kv, D, past=None):
    q = O.fill_normal(seed, n_head * n_q, D).reshape(n_head, n_q, D)
    k = O.fill_normal(seed + 1, n_kv_head * n_kv, D).reshape(n_kv_head, n_kv, D).astype(np.float16).view(np.uint16)
    v = O.fill_normal(seed + 2, n_kv_head * n_kv, D).reshape(n_kv_head, n_kv, D).astype(np.float16).view(np.uint16)
    mask = None
    if past is not None:
        m = np.zeros((n_q, n_kv), np.float32)
        for i in range(n_q):
            m[i, past + i + 1:] = -np.inf
        mask = m.astype(np.float16).view(np.uint16)
    return q, k, v, mask


@pytest.mark.parametrize("n_head,n_kv_head,n_q,n_kv,D,past", [(16, 8, 1, 256, 128, 200), (4, 2, 9, 64, 64, 40),
                                                              (2, 2, 3, 100, 128, None)])
def test_flash_attn_against_float64(n_head, n_kv_head, n_q, n_kv, D, past):
    q, k, v, mask = fa_case(11 + D + n_q, n_head, n_kv_head, n_q, n_kv, D, past)
    scale = 1.0 / np.sqrt(D)
    ref = attn_numpy(q, k, v, mask, scale)
    exact = O.flash_attn_ext(q, k, v, mask, scale, exact=True)
    assert np.abs(exact - ref).max() <= 1e-6 * np.abs(ref).max()
    cpu = O.flash_attn_ext(q, k, v, mask, scale)
    # ggml-cpu's loop keeps the V accumulator in fp16: within a few fp16 ulps of the exact attention
    assert np.abs(cpu - ref).max() <= 1e-2 * np.abs(ref).max()


@pytest.mark.parametrize("threads", [1, 4])
def test_cpu_port_flash_attn_against_float64(threads):
    """The multi-threaded F16C port timed as the whole decode step's CPU baseline (fp16 V accumulator, as ggml-cpu)
    holds the oracle's bar against the float64 attention, at the decode step's shape (16 q heads over 8 kv heads, one
    row, 1025 of 1088 positions visible) and with several rows."""
    for n_head, n_kv_head, n_q, n_kv, D, past in ((16, 8, 1, 1088, 128, 1024), (4, 2, 9, 64, 64, 40)):
        q, k, v, mask = fa_case(41 + n_q, n_head, n_kv_head, n_q, n_kv, D, past)
        ref = attn_numpy(q, k, v, mask, 1.0 / np.sqrt(D))
        got = O.cpu_fast_flash_attn_ext(q, k, v, mask, 1.0 / np.sqrt(D), threads)
        assert np.abs(got - ref).max() <= 1e-2 * np.abs(ref).max()
        assert np.abs(got - O.flash_attn_ext(q, k, v, mask, 1.0 / np.sqrt(D))).max() <= 1e-2 * np.abs(ref).max()


def test_flash_attn_closed_forms():
    D = 64
    q, k, v, _ = fa_case(21, 2, 1, 2, 64, D)
    # only position 5 visible: the output is V row 5
    m = np.full((2, 64), -np.inf, np.float32)
    m[:, 5] = 0
    out = O.flash_attn_ext(q, k, v, m.astype(np.float16).view(np.uint16), 0.125, exact=True)
    assert np.allclose(out, v[0, 5].view(np.float16).astype(np.float32)[None, None], atol=0)
    # q = 0: uniform scores, the output is the mean of the visible V rows
    out = O.flash_attn_ext(np.zeros_like(q), k, v, None, 0.125)
    mean = v[0].view(np.float16).astype(np.float64).mean(axis=0)
    assert np.abs(out - mean).max() <= 2e-3
    # everything masked: zeros (S = 0)
    allm = np.full((2, 64), -np.inf, np.float32).astype(np.float16).view(np.uint16)
    assert not O.flash_attn_ext(q, k, v, allm, 0.125).any()


def test_flash_attn_mutations_fail():
    q, k, v, mask = fa_case(31, 4, 2, 3, 64, 64, 40)
    ref = attn_numpy(q, k, v, mask, 0.125)
    # another scale, or reading kv head h % n_kv_head instead of h // group, is far off
    assert np.abs(O.flash_attn_ext(q, k, v, mask, 0.25, exact=True) - ref).max() > 1e-2
    k2 = k[[0, 1]].copy()
    alt = attn_numpy(q[[0, 2, 1, 3]], k2, v, mask, 0.125)[:, [0, 2, 1, 3]]
    assert np.abs(alt - ref).max() > 1e-2
