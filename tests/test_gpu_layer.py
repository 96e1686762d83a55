"""The decoder layer's other ops on MI355X against the oracle: RMS_NORM (alone and with the norm weight fused),
ADD / MUL, SWIGLU, ROPE NEOX, SET_ROWS into the f16 cache, and FLASH_ATTN_EXT over cache views as the decoder builds
them (qwen3-decoder.cpp:350-410).

Bars: SET_ROWS, ADD and MUL bit-exact; RMS_NORM within one float ulp (the CPU sums in double; so does the kernel, in
another order); SWIGLU and ROPE within 2e-6 (expf / sinf / cosf of the device's math library); FLASH_ATTN_EXT within
1e-5 of the row's largest output against the exact attention (fp32 V sum, as the graph's GGML_PREC_F32 asks), and
no further from ggml-cpu's own loop, whose V accumulator is fp16, than that loop is from the exact attention."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def dev(mx, be, x, t=None):
    x = np.ascontiguousarray(x)
    t = t if t is not None else mx.F32
    return be.tensor(t, tuple(reversed(x.shape)), x)


def out(mx, be, shape):
    return be.tensor(mx.F32, tuple(reversed(shape)))


def ulps(a, b):
    ai = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
    bi = np.ascontiguousarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(ai - bi).max()


@pytest.mark.parametrize("shape", [(7, 1024), (3, 16, 128), (2, 2048)])
def test_rms_norm(mx, be, shape):
    x = O.fill_normal(0x1A00 + shape[-1], int(np.prod(shape[:-1])), shape[-1]).reshape(shape)
    X, Y = dev(mx, be, x), out(mx, be, shape)
    be.rms_norm(X, Y, 1e-6)
    be.sync()
    ref = O.rms_norm(x, 1e-6)
    got = Y.numpy().reshape(shape)
    assert ulps(got, ref) <= 1
    w = O.fill_normal(0x1B00, 1, shape[-1])[0]
    W, Z = dev(mx, be, w), out(mx, be, shape)
    be.rms_norm(X, Z, 1e-6, W)
    be.sync()
    assert ulps(Z.numpy().reshape(shape), O.binary("mul", ref, w)) <= 2


def test_add_mul_broadcast(mx, be):
    a = O.fill_normal(0x1C00, 6, 1024)
    for b in (O.fill_normal(0x1C01, 1, 1024), O.fill_normal(0x1C02, 3, 1024), O.fill_normal(0x1C03, 6, 1024)):
        A, B = dev(mx, be, a), dev(mx, be, b)
        for op, fn in (("add", be.add), ("mul", be.mul)):
            Y = out(mx, be, a.shape)
            fn(A, B, Y)
            be.sync()
            assert np.array_equal(Y.numpy().reshape(a.shape), O.binary(op, a, b))


def test_swiglu(mx, be):
    a = O.fill_normal(0x1D00, 5, 3072) * np.float32(4)
    b = O.fill_normal(0x1D01, 5, 3072)
    A, B, Y = dev(mx, be, a), dev(mx, be, b), out(mx, be, a.shape)
    be.swiglu(A, B, Y)
    be.sync()
    ref = O.swiglu(a, b)
    assert np.abs(Y.numpy().reshape(a.shape) - ref).max() <= 2e-6 * np.abs(ref).max()


@pytest.mark.parametrize("n_dims", [128, 64])
def test_rope_neox(mx, be, n_dims):
    rows, heads, D = 6, 16, 128
    x = O.fill_normal(0x1E00, rows * heads, D).reshape(rows, heads, D)
    pos = np.array([0, 1, 37, 1000, 4095, 70000], np.int32)
    X, P, Y = dev(mx, be, x), dev(mx, be, pos, mx.I32), out(mx, be, x.shape)
    be.rope(X, P, Y, n_dims, 1e6)
    be.sync()
    ref = O.rope_neox(x, pos, n_dims, 1e6)
    assert np.abs(Y.numpy().reshape(x.shape) - ref).max() <= 2e-6


def test_set_rows_into_f16_cache(mx, be):
    kv_dim, cap = 1024, 64
    cache = (O.fill_normal(0x1F00, cap, kv_dim)).astype(np.float16).view(np.uint16)
    src = O.fill_normal(0x1F01, 3, kv_dim) * np.float32(50)
    idx = np.array([63, 0, 17], np.int32)
    C = dev(mx, be, cache, mx.F16)
    S, I = dev(mx, be, src), dev(mx, be, idx, mx.I32)
    be.set_rows(S, I, C)
    be.sync()
    got = np.frombuffer(C.get_bytes().tobytes(), np.uint16).reshape(cap, kv_dim)
    assert np.array_equal(got, O.set_rows_f16(cache, src, idx))
    bad = dev(mx, be, np.array([5, cap, 1], np.int32), mx.I32)
    be.set_rows(S, bad, C)
    with pytest.raises(mx.MxError) as e:
        be.sync()
    assert e.value.code == mx.INVALID
    got2 = np.frombuffer(C.get_bytes().tobytes(), np.uint16).reshape(cap, kv_dim)
    want = O.set_rows_f16(O.set_rows_f16(cache, src, idx), src[[0, 2]], np.array([5, 1], np.int32))
    assert np.array_equal(got2, want)


def fa_device(mx, be, n_head, n_kv_head, n_q, n_kv, cap, D, past, seed):
    """q, K / V and mask laid out as Qwen3Decoder::layers builds them: q [D, n_head, n_q] read through
    permute(0, 2, 1, 3); the f16 caches [n_kv_head * D, cap] read through view_3d + permute; the mask [n_kv, n_q]."""
    q = O.fill_normal(seed, n_q * n_head, D).reshape(n_q, n_head, D)
    kc = O.fill_normal(seed + 1, cap, n_kv_head * D).astype(np.float16).view(np.uint16).reshape(cap, n_kv_head, D)
    vc = O.fill_normal(seed + 2, cap, n_kv_head * D).astype(np.float16).view(np.uint16).reshape(cap, n_kv_head, D)
    m = np.zeros((n_q, n_kv), np.float32)
    for i in range(n_q):
        m[i, past + i + 1:] = -np.inf
    mask = m.astype(np.float16).view(np.uint16)
    Q = dev(mx, be, q)
    K = dev(mx, be, kc, mx.F16)
    V = dev(mx, be, vc, mx.F16)
    M = dev(mx, be, mask, mx.F16)
    kv_dim = n_kv_head * D
    qh = Q.view((D, n_q, n_head), (4, n_head * D * 4, D * 4))
    kh = K.view((D, n_kv, n_kv_head), (2, kv_dim * 2, D * 2))
    vh = V.view((D, n_kv, n_kv_head), (2, kv_dim * 2, D * 2))
    O_ = be.tensor(mx.F32, (D, n_head, n_q))
    args = (q.transpose(1, 0, 2), kc[:n_kv].transpose(1, 0, 2), vc[:n_kv].transpose(1, 0, 2), mask)
    return (qh, kh, vh, M, O_), args


@pytest.mark.parametrize("n_head,n_kv_head,n_q,n_kv,cap,D,past", [
    (16, 8, 1, 1024, 1280, 128, 1000),    # a 0.6B decode step: 1001 positions, read as 16 blocks of 64
    (16, 8, 1, 64, 256, 128, 0),          # the first token
    (16, 8, 40, 576, 640, 128, 530),      # a prefill block after earlier blocks
    (8, 2, 5, 192, 192, 64, 150),         # head size 64, four heads per kv head
    (8, 8, 3, 130, 192, 128, 127),        # one q head per kv head, 130 positions (a ragged last block)
    (16, 4, 2, 300, 320, 128, 298),       # four q heads per kv head
])
def test_flash_attn_ext(mx, be, n_head, n_kv_head, n_q, n_kv, cap, D, past):
    (qh, kh, vh, M, Y), (q, k, v, mask) = fa_device(mx, be, n_head, n_kv_head, n_q, n_kv, cap, D, past,
                                                    0x2A00 + n_q + D)
    scale = 1.0 / np.sqrt(D)
    assert mx.lib().mx_supports_flash_attn_ext(qh.ref(), kh.ref(), vh.ref(), M.ref(), Y.ref(), 0.0, 0.0)
    be.flash_attn_ext(qh, kh, vh, M, Y, scale)
    be.sync()
    got = Y.numpy().reshape(n_q, n_head, D)
    exact = O.flash_attn_ext(q, k, v, mask, scale, exact=True)
    cpu = O.flash_attn_ext(q, k, v, mask, scale)
    big = np.abs(exact).max(axis=2, keepdims=True)
    assert (np.abs(got - exact) / big).max() <= 1e-5
    # ggml-cpu's loop rounds its V accumulator to fp16 at every position (1.4 % of the row's largest output after
    # 1000 positions): the device is never further from it than it is from the exact attention
    cpu_dev = (np.abs(cpu - exact) / big).max()
    assert (np.abs(got - cpu) / big).max() <= cpu_dev + 1e-5
    # again: whichever split's workgroup merges, the result is the same bits (and the merge counts start from zero)
    for _ in range(2):
        be.flash_attn_ext(qh, kh, vh, M, Y, scale)
        be.sync()
        assert np.array_equal(Y.numpy().reshape(n_q, n_head, D), got)


def test_flash_attn_no_positions_or_rows(mx, be):
    """A K / V view of no positions: every output row is zero (ggml-cpu's S = 0 case); no query rows: nothing is
    written. Neither reaches the split arithmetic with a zero divisor."""
    D, n_head, n_kv_head, n_q = 128, 4, 2, 3
    K = be.tensor(mx.F16, (n_kv_head * D, 8))
    kh = K.view((D, 0, n_kv_head), (2, n_kv_head * D * 2, D * 2))
    q = O.fill_normal(0x2C00, n_q * n_head, D)
    Q = dev(mx, be, q)
    qh = Q.view((D, n_q, n_head), (4, n_head * D * 4, D * 4))
    Y = be.tensor(mx.F32, (D, n_head, n_q), np.full(n_q * n_head * D, 7.0, np.float32))
    be.flash_attn_ext(qh, kh, kh, None, Y, 0.1)
    be.sync()
    assert not Y.numpy().any()
    Y0 = Y.view((D, n_head, 0), (4, D * 4, n_head * D * 4))
    be.flash_attn_ext(Q.view((D, 0, n_head), (4, n_head * D * 4, D * 4)), kh, kh, None, Y0, 0.1)
    be.sync()


def test_flash_attn_unsupported_forms(mx, be):
    (qh, kh, vh, M, Y), _ = fa_device(mx, be, 4, 2, 1, 64, 64, 128, 10, 0x2B00)
    L = mx.lib()
    assert not L.mx_supports_flash_attn_ext(qh.ref(), kh.ref(), vh.ref(), M.ref(), Y.ref(), 8.0, 0.0)   # ALiBi
    assert not L.mx_supports_flash_attn_ext(qh.ref(), kh.ref(), vh.ref(), M.ref(), Y.ref(), 0.0, 30.0)  # softcap
    with pytest.raises(mx.MxError) as e:
        mx.check(L.mx_flash_attn_ext(be.h, qh.ref(), kh.ref(), kh.ref(), M.ref(), qh.ref(), 0.1))
    assert e.value.code == mx.UNSUPPORTED


def test_decoder_layers_chain(mx, be):
    """Two Qwen3-style layers (hidden 256, 4 q / 2 kv heads of 64, FFN 512, Q8_0 linears, an f16 cache holding 70
    positions) run op by op on the device as Qwen3Decoder::layers orders them, against the same chain in the oracle
    (attention in its exact form): the residual stream after both layers within 1e-4 of its largest value."""
    H, F, nq, nkv, hd, past, cap, eps, theta = 256, 512, 4, 2, 64, 70, 128, 1e-6, 1e6
    kv_dim, n_kv = nkv * hd, 128
    t = O.TYPE_Q8_0
    shapes = [("q", H, nq * hd), ("k", H, kv_dim), ("v", H, kv_dim), ("o", nq * hd, H), ("gate", H, F), ("up", H, F),
              ("down", F, H)]
    layers = []
    for l in range(2):
        ws = {n: O.quantize_chunk(t, O.fill_normal(0x3A00 + 16 * l + i, N, K, 0.0, 0.05))
              for i, (n, K, N) in enumerate(shapes)}
        nw = {n: O.fill_normal(0x3B00 + 16 * l + i, 1, k, 1.0, 0.1)[0]
              for i, (n, k) in enumerate([("attn", H), ("ffn", H), ("q", hd), ("k", hd)])}
        cache = {n: np.zeros((cap, kv_dim), np.uint16) for n in ("k", "v")}
        for j, n in enumerate(("k", "v")):
            cache[n][:past] = O.fill_normal(0x3C00 + 2 * l + j, past, kv_dim).astype(np.float16).view(np.uint16)
        layers.append((ws, nw, cache))
    x0 = O.fill_normal(0x3D00, 1, H)
    pos = np.array([past], np.int32)
    m = np.zeros((1, n_kv), np.float32)
    m[0, past + 1:] = -np.inf
    mask = m.astype(np.float16).view(np.uint16)

    # oracle chain
    x = x0.copy()
    for ws, nw, cache in layers:
        h = O.binary("mul", O.rms_norm(x, eps), nw["attn"])
        q, k, v = (O.mul_mat(t, ws[n], h) for n in ("q", "k", "v"))
        q = O.rope_neox(O.binary("mul", O.rms_norm(q.reshape(1, nq, hd), eps), nw["q"]), pos, hd, theta)
        k = O.rope_neox(O.binary("mul", O.rms_norm(k.reshape(1, nkv, hd), eps), nw["k"]), pos, hd, theta)
        kc = O.set_rows_f16(cache["k"], k.reshape(1, kv_dim), pos)[:n_kv].reshape(n_kv, nkv, hd).transpose(1, 0, 2)
        vc = O.set_rows_f16(cache["v"], v.reshape(1, kv_dim), pos)[:n_kv].reshape(n_kv, nkv, hd).transpose(1, 0, 2)
        att = O.flash_attn_ext(q.transpose(1, 0, 2), kc, vc, mask, 1.0 / np.sqrt(hd), exact=True)
        x = O.binary("add", x, O.mul_mat(t, ws["o"], att.reshape(1, -1)))
        h = O.binary("mul", O.rms_norm(x, eps), nw["ffn"])
        x = O.binary("add", x, O.mul_mat(t, ws["down"], O.swiglu(O.mul_mat(t, ws["gate"], h),
                                                                O.mul_mat(t, ws["up"], h))))
    # device chain
    X = dev(mx, be, x0)
    Hd = out(mx, be, (1, H))
    P = dev(mx, be, pos, mx.I32)
    M = dev(mx, be, mask, mx.F16)
    for ws, nw, cache in layers:
        W = {n: be.tensor(t, (K, N), ws[n]) for n, K, N in shapes}
        NW = {n: dev(mx, be, v) for n, v in nw.items()}
        C = {n: dev(mx, be, cache[n], mx.F16) for n in ("k", "v")}
        Y = {n: be.tensor(mx.F32, (N, 1)) for n, _, N in shapes}
        qn, qr = be.tensor(mx.F32, (hd, nq, 1)), be.tensor(mx.F32, (hd, nq, 1))
        kn, kr = be.tensor(mx.F32, (hd, nkv, 1)), be.tensor(mx.F32, (hd, nkv, 1))
        att = be.tensor(mx.F32, (hd, nq, 1))
        act = be.tensor(mx.F32, (F, 1))
        be.rms_norm(X, Hd, eps, NW["attn"])
        be.mul_mat_group([W["q"], W["k"], W["v"]], Hd, [Y["q"], Y["k"], Y["v"]])
        be.rms_norm(Y["q"].view((hd, nq, 1), (4, hd * 4, nq * hd * 4)), qn, eps, NW["q"])
        be.rms_norm(Y["k"].view((hd, nkv, 1), (4, hd * 4, kv_dim * 4)), kn, eps, NW["k"])
        be.set_rows(Y["v"], P, C["v"])
        be.rope(qn, P, qr, hd, theta)
        be.rope(kn, P, kr, hd, theta)
        be.set_rows(kr.view((kv_dim, 1), (4, kv_dim * 4)), P, C["k"])
        be.flash_attn_ext(qr.view((hd, 1, nq), (4, nq * hd * 4, hd * 4)),
                          C["k"].view((hd, n_kv, nkv), (2, kv_dim * 2, hd * 2)),
                          C["v"].view((hd, n_kv, nkv), (2, kv_dim * 2, hd * 2)), M, att, 1.0 / np.sqrt(hd))
        be.mul_mat(W["o"], att.view((nq * hd, 1), (4, nq * hd * 4)), Y["o"])
        be.add(X, Y["o"], X)
        be.rms_norm(X, Hd, eps, NW["ffn"])
        be.mul_mat_group([W["gate"], W["up"]], Hd, [Y["gate"], Y["up"]])
        be.swiglu(Y["gate"], Y["up"], act)
        be.mul_mat(W["down"], act, Y["down"])
        be.add(X, Y["down"], X)
        be.sync()
    got = X.numpy().reshape(1, H)
    assert np.abs(got - x).max() <= 1e-4 * np.abs(x).max()


def test_fused_products_equal_the_separate_ops(mx, be):
    """mul(rms_norm) before q/k/v, swiglu before down and the residual add after it, fused into the mat-vec: the
    same bits as the separate ops, and within the products' bar of the oracle."""
    H, F, t, eps = 1024, 3072, O.TYPE_Q8_0, 1e-6
    wq = [O.quantize_chunk(t, O.fill_normal(0x4A00 + i, n, H, 0.0, 0.02)) for i, n in enumerate((2048, 1024, 1024))]
    wd = O.quantize_chunk(t, O.fill_normal(0x4A10, H, F, 0.0, 0.02))
    x = O.fill_normal(0x4A20, 1, H) * np.float32(3)
    nw = O.fill_normal(0x4A21, 1, H, 1.0, 0.1)[0]
    g, u = O.fill_normal(0x4A22, 1, F), O.fill_normal(0x4A23, 1, F)
    X, NW, G, U = dev(mx, be, x), dev(mx, be, nw), dev(mx, be, g), dev(mx, be, u)
    WQ = [be.tensor(t, (H, w.shape[0]), w) for w in wq]
    WD = be.tensor(t, (F, H), wd)
    # separate ops
    Hn = out(mx, be, (1, H))
    be.rms_norm(X, Hn, eps, NW)
    Ys = [out(mx, be, (1, w.shape[0])) for w in wq]
    be.mul_mat_group(WQ, Hn, Ys)
    A = out(mx, be, (1, F))
    be.swiglu(G, U, A)
    D = out(mx, be, (1, H))
    be.mul_mat(WD, A, D)
    R = dev(mx, be, x)
    be.add(R, D, R)
    # fused
    Yf = [out(mx, be, (1, w.shape[0])) for w in wq]
    be.mul_mat_fused(WQ, X, Yf, norm_w=NW, eps=eps)
    Rf = dev(mx, be, x)
    be.mul_mat_fused([WD], G, [Rf], glu_b=U, residual=[Rf])
    be.sync()
    for ys, yf in zip(Ys, Yf):
        assert np.array_equal(ys.numpy(), yf.numpy())
    assert np.array_equal(R.numpy(), Rf.numpy())
    h = O.binary("mul", O.rms_norm(x, eps), nw)
    for w, yf in zip(wq, Yf):
        assert rel_err_rows(yf.numpy().reshape(1, -1), O.mul_mat(t, w, h)) <= 2e-5
    ref = O.binary("add", x, O.mul_mat(t, wd, O.swiglu(g, u)))
    assert np.abs(Rf.numpy().reshape(1, H) - ref).max() <= 2e-5 * np.abs(ref).max()


def rel_err_rows(y, ref):
    return float((np.abs(y - ref).max(axis=1) / np.abs(ref).max(axis=1)).max())


def test_fused_qk_norm_rope_kv_equals_the_separate_ops(mx, be):
    nq, nkv, hd, cap, eps, theta = 16, 8, 128, 96, 1e-6, 1e6
    kv_dim = nkv * hd
    q = O.fill_normal(0x4B00, 1, nq * hd) * np.float32(2)
    k = O.fill_normal(0x4B01, 1, kv_dim)
    v = O.fill_normal(0x4B02, 1, kv_dim)
    qw, kw = O.fill_normal(0x4B03, 1, hd, 1.0, 0.1)[0], O.fill_normal(0x4B04, 1, hd, 1.0, 0.1)[0]
    pos = np.array([77], np.int32)
    cache0 = O.fill_normal(0x4B05, cap, kv_dim).astype(np.float16).view(np.uint16)
    Q, K, V, QW, KW, P = dev(mx, be, q), dev(mx, be, k), dev(mx, be, v), dev(mx, be, qw), dev(mx, be, kw), \
        dev(mx, be, pos, mx.I32)
    qv = Q.view((hd, nq, 1), (4, hd * 4, nq * hd * 4))
    kv = K.view((hd, nkv, 1), (4, hd * 4, kv_dim * 4))
    vv = V.view((hd, nkv, 1), (4, hd * 4, kv_dim * 4))
    # separate ops
    KC, VC = dev(mx, be, cache0, mx.F16), dev(mx, be, cache0, mx.F16)
    qn, kn = be.tensor(mx.F32, (hd, nq, 1)), be.tensor(mx.F32, (hd, nkv, 1))
    qr, kr = be.tensor(mx.F32, (hd, nq, 1)), be.tensor(mx.F32, (hd, nkv, 1))
    be.rms_norm(qv, qn, eps, QW)
    be.rms_norm(kv, kn, eps, KW)
    be.set_rows(V, P, VC)
    be.rope(qn, P, qr, hd, theta)
    be.rope(kn, P, kr, hd, theta)
    be.set_rows(kr.view((kv_dim, 1), (4, kv_dim * 4)), P, KC)
    # fused
    KC2, VC2 = dev(mx, be, cache0, mx.F16), dev(mx, be, cache0, mx.F16)
    qo = be.tensor(mx.F32, (hd, nq, 1))
    be.qk_norm_rope_kv(qv, kv, vv, QW, KW, P, qo, KC2, VC2, eps, theta)
    be.sync()
    assert np.array_equal(qo.numpy(), qr.numpy())
    assert np.array_equal(KC2.get_bytes(), KC.get_bytes())
    assert np.array_equal(VC2.get_bytes(), VC.get_bytes())
    ref_q = O.rope_neox(O.binary("mul", O.rms_norm(q.reshape(1, nq, hd), eps), qw), pos, hd, theta)
    assert np.abs(qo.numpy().reshape(1, nq, hd) - ref_q).max() <= 2e-6


@pytest.mark.parametrize("nq,nkv,p,n_kv,masked", [
    (16, 8, 1000, 1088, True),   # a 0.6B decode step: the new row inside the last split
    (8, 8, 63, 64, True),        # one q head per kv head, the new row last of a single chunk
    (16, 4, 130, 256, True),     # four q heads per kv head, the new row first of the third chunk
    (16, 8, 300, 256, True),     # the new row past the positions read: stored, not attended
    (16, 8, 700, 701, False),    # no mask: every position read is visible (a ragged last chunk)
])
def test_attn_decode_equals_the_separate_ops(mx, be, nq, nkv, p, n_kv, masked):
    """mx_attn_decode gives the bits of mx_qk_norm_rope_kv followed by mx_flash_attn_ext: the output and both
    caches."""
    hd, cap, eps, theta = 128, 320 if n_kv < 320 else 1280, 1e-6, 1e6
    kv_dim = nkv * hd
    seed = 0x4C00 + nq + nkv + p
    q = O.fill_normal(seed, 1, nq * hd) * np.float32(2)
    k = O.fill_normal(seed + 1, 1, kv_dim)
    v = O.fill_normal(seed + 2, 1, kv_dim)
    qw, kw = O.fill_normal(seed + 3, 1, hd, 1.0, 0.1)[0], O.fill_normal(seed + 4, 1, hd, 1.0, 0.1)[0]
    pos = np.array([p], np.int32)
    cache0 = O.fill_normal(seed + 5, cap, kv_dim).astype(np.float16).view(np.uint16)
    m = np.zeros((1, n_kv), np.float32)
    m[0, p + 1:] = -np.inf
    mask = m.astype(np.float16).view(np.uint16)
    Q, K, V, QW, KW, P = dev(mx, be, q), dev(mx, be, k), dev(mx, be, v), dev(mx, be, qw), dev(mx, be, kw), \
        dev(mx, be, pos, mx.I32)
    M = dev(mx, be, mask, mx.F16) if masked else None
    qv = Q.view((hd, nq, 1), (4, hd * 4, nq * hd * 4))
    kv = K.view((hd, nkv, 1), (4, hd * 4, kv_dim * 4))
    vv = V.view((hd, nkv, 1), (4, hd * 4, kv_dim * 4))
    scale = 1.0 / np.sqrt(hd)

    def views(KC, VC):
        return (KC.view((hd, n_kv, nkv), (2, kv_dim * 2, hd * 2)), VC.view((hd, n_kv, nkv), (2, kv_dim * 2, hd * 2)))

    KC, VC = dev(mx, be, cache0, mx.F16), dev(mx, be, cache0, mx.F16)
    qo = be.tensor(mx.F32, (hd, nq, 1))
    Y = be.tensor(mx.F32, (hd, nq, 1))
    be.qk_norm_rope_kv(qv, kv, vv, QW, KW, P, qo, KC, VC, eps, theta)
    kh, vh = views(KC, VC)
    be.flash_attn_ext(qo.view((hd, 1, nq), (4, nq * hd * 4, hd * 4)), kh, vh, M, Y, scale)
    KC2, VC2 = dev(mx, be, cache0, mx.F16), dev(mx, be, cache0, mx.F16)
    Y2 = be.tensor(mx.F32, (hd, nq, 1))
    kh2, vh2 = views(KC2, VC2)
    be.attn_decode(qv, kv, vv, QW, KW, P, KC2, VC2, kh2, vh2, M, Y2, eps, theta, scale)
    be.sync()
    assert np.array_equal(KC2.get_bytes(), KC.get_bytes())
    assert np.array_equal(VC2.get_bytes(), VC.get_bytes())
    y, y2 = Y.numpy().reshape(nq, hd), Y2.numpy().reshape(nq, hd)
    diff = np.argwhere(y.view(np.uint32) != y2.view(np.uint32))
    assert len(diff) == 0, (len(diff), diff[:8].tolist(), float(np.abs(y - y2).max()))


def test_attn_decode_unsupported_forms(mx, be):
    """Two rows, views that do not start at cache row 0, or a group of three q heads per kv head: MX_UNSUPPORTED
    (the caller runs mx_qk_norm_rope_kv and mx_flash_attn_ext instead); nothing is launched."""
    hd, nkv, cap, n_kv = 128, 2, 128, 64
    kv_dim = nkv * hd
    L = mx.lib()

    def case(nq, rows, view_row0):
        Q = be.tensor(mx.F32, (hd, nq, rows))
        K = be.tensor(mx.F32, (hd, nkv, rows))
        V = be.tensor(mx.F32, (hd, nkv, rows))
        W = be.tensor(mx.F32, (hd,))
        P = be.tensor(mx.I32, (rows,), np.arange(rows, dtype=np.int32))
        KC, VC = be.tensor(mx.F16, (kv_dim, cap)), be.tensor(mx.F16, (kv_dim, cap))
        off = view_row0 * kv_dim * 2
        kh = KC.view((hd, n_kv, nkv), (2, kv_dim * 2, hd * 2), off)
        vh = VC.view((hd, n_kv, nkv), (2, kv_dim * 2, hd * 2), off)
        Y = be.tensor(mx.F32, (hd, nq, rows))
        return L.mx_attn_decode(be.h, Q.ref(), K.ref(), V.ref(), W.ref(), W.ref(), P.ref(), KC.ref(), VC.ref(),
                                kh.ref(), vh.ref(), None, Y.ref(), 1e-6, 128, mx.ROPE_NEOX, 1e6, 1.0, 0.0, 1.0, 0.1)

    assert case(4, 1, 0) == 0            # the supported form, for contrast (no mask: every position visible)
    assert case(4, 2, 0) == mx.UNSUPPORTED
    assert case(4, 1, 8) == mx.UNSUPPORTED
    assert case(6, 1, 0) == mx.UNSUPPORTED
    be.sync()
