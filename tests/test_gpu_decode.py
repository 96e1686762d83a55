"""Skipped: the one-launch decode step these tests held (mx_decoder_new / mx_decoder_step: Qwen3Decoder::step as one
persistent launch) was taken out of the library after its first GPU run faulted with no cause shown. They checked it
against
the oracle's chain of the same ops (GET_ROWS, per layer RMS_NORM x weight, q/k/v, q/k norms, NEOX RoPE, SET_ROWS into
the f16 caches, exact flash attention over positions 0..p, attn_o + residual, RMS_NORM, gate/up, SwiGLU, down +
residual; final norm, output head, ARGMAX), on the 0.6B shape's layers (hidden 1024, 16 q / 8 kv heads of 128, FFN
3072) with two layers and a 5000-row head. Bars: the new cache rows within one fp16 ulp of the oracle's (the k / v
products differ from it only in fp32 summation order), logits within 1e-4 of the largest |logit| (the bar the
layer chain holds), and the pick the oracle's argmax (or a logit within that bar of the oracle's maximum)."""
import numpy as np
import pytest

import oracle as O

pytestmark = [pytest.mark.gpu,
              pytest.mark.skip(reason="the one-launch decode step was taken out of the library: its first run faulted "
                                      "the GPU and the cause was not found")]

Q8 = O.TYPE_Q8_0
H, F, NQ, NKV, HD, V, EPS, THETA = 1024, 3072, 16, 8, 128, 5000, 1e-6, 1e6
KV = NKV * HD
SHAPES = [("wq", H, NQ * HD), ("wk", H, KV), ("wv", H, KV), ("wo", NQ * HD, H), ("w_gate", H, F), ("w_up", H, F),
          ("w_down", F, H)]


def make_model(mx, be, n_layer, cap, past, seed):
    """Host copies and device tensors of a random-init model with f16 caches holding N(0,1) values at rows < past."""
    host, dev_layers = [], []
    for l in range(n_layer):
        h = {n: mx.quantize_normal(Q8, seed + 32 * l + i, N, K, 0.02) for i, (n, K, N) in enumerate(SHAPES)}
        for i, (n, k) in enumerate([("attn_norm", H), ("ffn_norm", H), ("q_norm", HD), ("k_norm", HD)]):
            h[n] = mx.fill_normal(seed + 32 * l + 16 + i, 1, k, 1.0, 0.1)[0]
        for j, n in enumerate(("k_cache", "v_cache")):
            c = np.zeros((cap, KV), np.uint16)
            c[:past] = mx.fill_normal(seed + 32 * l + 24 + j, past, KV).astype(np.float16).view(np.uint16)
            h[n] = c
        host.append(h)
        d = {n: be.tensor(Q8, (K, N), h[n]) for n, K, N in SHAPES}
        for n in ("attn_norm", "ffn_norm", "q_norm", "k_norm"):
            d[n] = be.tensor(mx.F32, (h[n].shape[0],), h[n])
        for n in ("k_cache", "v_cache"):
            d[n] = be.tensor(mx.F16, (KV, cap), h[n])
        dev_layers.append(d)
    emb = mx.quantize_normal(Q8, seed + 999, V, H, 0.02)
    onorm = mx.fill_normal(seed + 998, 1, H, 1.0, 0.1)[0]
    E, ON = be.tensor(Q8, (H, V), emb), be.tensor(mx.F32, (H,), onorm)
    dec = be.decoder(dev_layers, E, ON, E, NQ, NKV, EPS, THETA)
    return dec, host, dev_layers, emb, onorm


def oracle_step(host, emb, onorm, tok, p):
    """The step in the oracle; updates the host caches' row p. Returns logits [V]."""
    x = O.get_rows(Q8, emb, H, np.array([tok], np.int32))
    pos = np.array([p], np.int32)
    for h in host:
        hn = O.binary("mul", O.rms_norm(x, EPS), h["attn_norm"])
        q, k, v = (O.mul_mat(Q8, h[n], hn) for n in ("wq", "wk", "wv"))
        q = O.rope_neox(O.binary("mul", O.rms_norm(q.reshape(1, NQ, HD), EPS), h["q_norm"]), pos, HD, THETA)
        k = O.rope_neox(O.binary("mul", O.rms_norm(k.reshape(1, NKV, HD), EPS), h["k_norm"]), pos, HD, THETA)
        h["k_cache"] = O.set_rows_f16(h["k_cache"], k.reshape(1, KV), pos)
        h["v_cache"] = O.set_rows_f16(h["v_cache"], v.reshape(1, KV), pos)
        kc = h["k_cache"][:p + 1].reshape(p + 1, NKV, HD).transpose(1, 0, 2)
        vc = h["v_cache"][:p + 1].reshape(p + 1, NKV, HD).transpose(1, 0, 2)
        att = O.flash_attn_ext(q.transpose(1, 0, 2), kc, vc, None, 1.0 / np.sqrt(HD), exact=True)
        x = O.binary("add", x, O.mul_mat(Q8, h["wo"], att.reshape(1, -1)))
        hn = O.binary("mul", O.rms_norm(x, EPS), h["ffn_norm"])
        x = O.binary("add", x, O.mul_mat(Q8, h["w_down"], O.swiglu(O.mul_mat(Q8, h["w_gate"], hn),
                                                                   O.mul_mat(Q8, h["w_up"], hn))))
    hn = O.binary("mul", O.rms_norm(x, EPS), onorm)
    return O.mul_mat(Q8, emb, hn)[0]


def f16_ulps(a, b):
    a = a.astype(np.int32)
    b = b.astype(np.int32)
    sa = np.where(a & 0x8000, 0x8000 - a, a)
    sb = np.where(b & 0x8000, 0x8000 - b, b)
    return int(np.abs(sa - sb).max())


def check_step(mx, dev_layers, host, logits, pick, ref, p):
    got = logits.numpy().reshape(-1)[:V]
    scale = np.abs(ref).max()
    assert np.abs(got - ref).max() <= 1e-4 * scale, f"logits off by {np.abs(got - ref).max() / scale:.3g}"
    k = int(pick.numpy().reshape(-1)[0])
    assert k == int(np.argmax(ref)) or ref[k] >= ref.max() - 1e-4 * scale
    for d, h in zip(dev_layers, host):
        for n in ("k_cache", "v_cache"):
            row = d[n].get_bytes(offset=p * KV * 2, size=KV * 2).view(np.uint16)
            assert f16_ulps(row, h[n][p]) <= 1, f"{n} row {p}"


@pytest.mark.parametrize("p", [1024, 5, 2100], ids=["p1024", "p5", "p2100"])
def test_decode_step_matches_the_oracle_chain(mx, be, p):
    """p = 1024: 33 positions per attention split (one chunk); p = 5: most splits empty; p = 2100: 66 positions per
    split (a second chunk read outside the prefetched one)."""
    dec, host, dev_layers, emb, onorm = make_model(mx, be, 2, 2304, p, 0x7E000 + p)
    tok = be.tensor(mx.I32, (1,), np.array([4321], np.int32))
    pos = be.tensor(mx.I32, (1,), np.array([p], np.int32))
    logits, pick = be.tensor(mx.F32, (V,)), be.tensor(mx.I32, (1,))
    try:
        dec.step(tok, pos, logits, pick)
        be.sync()
        ref = oracle_step(host, emb, onorm, 4321, p)
        check_step(mx, dev_layers, host, logits, pick, ref, p)
    finally:
        dec.free()


def test_decode_steps_chain_through_the_pick(mx, be):
    """Three steps in a row, each fed the previous step's pick on the device (no host round trip): each step reads the
    cache rows the steps before it wrote, and its tags differ from theirs."""
    p0 = 700
    dec, host, dev_layers, emb, onorm = make_model(mx, be, 2, 1024, p0, 0x7E100)
    tok = be.tensor(mx.I32, (1,), np.array([17], np.int32))
    logits, pick = be.tensor(mx.F32, (V,)), be.tensor(mx.I32, (1,))
    picks = [be.tensor(mx.I32, (1,)) for _ in range(3)]
    try:
        t_host = 17
        src = tok
        for i in range(3):
            p = p0 + i
            pos = be.tensor(mx.I32, (1,), np.array([p], np.int32))
            dec.step(src, pos, logits, picks[i])
            be.sync()
            ref = oracle_step(host, emb, onorm, t_host, p)
            check_step(mx, dev_layers, host, logits, picks[i], ref, p)
            t_host = int(picks[i].numpy().reshape(-1)[0])
            src = picks[i]
    finally:
        dec.free()


def test_decode_step_refusals(mx, be):
    """A position outside the caches is reported by the next synchronize and computes nothing; a model the step
    kernel does not take is refused when the decoder is made."""
    dec, host, dev_layers, emb, onorm = make_model(mx, be, 1, 64, 10, 0x7E200)
    tok = be.tensor(mx.I32, (1,), np.array([3], np.int32))
    bad = be.tensor(mx.I32, (1,), np.array([64], np.int32))
    logits, pick = be.tensor(mx.F32, (V,)), be.tensor(mx.I32, (1,))
    try:
        dec.step(tok, bad, logits, pick)
        with pytest.raises(mx.MxError) as e:
            be.sync()
        assert e.value.code == mx.INVALID
        be.sync()
    finally:
        dec.free()
    d0 = dev_layers[0]
    q4 = be.tensor(mx.Q4_K, (H, NQ * HD))
    layer = dict(d0, wq=q4)
    with pytest.raises(mx.MxError) as e:
        be.decoder([layer], d0["wq"], d0["attn_norm"], d0["wq"], NQ, NKV, EPS, THETA)
    assert e.value.code == mx.UNSUPPORTED
