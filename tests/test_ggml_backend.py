"""The ggml backend (speech.cpp_amd/libggml-mi355x.so) driven through ggml's own API, as speech.cpp drives a backend:
registry -> device -> buffer type -> buffers -> tensors uploaded in 16 MB pieces -> graphs built with ggml's op
constructors -> ggml_backend_graph_compute (src/common/backend.cpp:70-120, model-file.cpp:222-268, graph.cpp:96-110,
qwen3-decoder.cpp:187-208,350-438). ggml itself is absent here: tests/ggml_host stands in for ggml's core and backend
dispatch.

Without a GPU: the library's exports, the registry and its check of the linked ggml (a ggml numbering its ops
differently registers no device), and the backend's plan of a Qwen3 decode graph (which nodes fuse).
On MI355X: a graph of a q/k/v group, GET_ROWS, MUL_MAT_ID and ARGMAX computed four times (eager twice, recorded,
replayed), and a two-layer Qwen3 decode graph over four steps with the fused kernels, each against the oracle."""
import ctypes
import pathlib
import subprocess
import sys
import textwrap

import numpy as np
import pytest

import ggml_graph as G
import oracle as O
from helpers import dq_model, rel_err
from test_gpu_layer import ulps

ROOT = pathlib.Path(__file__).resolve().parents[1]
TIGHT = 2e-5  # the products' bar on the integer paths (exact per-block sums, fp32 cross-block sums)


# --------------------------------------------------------------------------------------------- without a GPU
def test_library_exports_the_registry_only():
    out = subprocess.run(["nm", "-D", "--defined-only", str(G.BACKEND_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = sorted(l.split()[-1] for l in out.splitlines() if " T " in l)
    assert exported == ["ggml_backend_init", "ggml_backend_mi355x_reg"]


def test_registry_and_linked_ggml_check():
    h, b = G.libs()
    reg = b.ggml_backend_mi355x_reg()
    assert h.ggml_backend_reg_name(reg) == b"MI355X"
    assert ctypes.cast(reg, ctypes.POINTER(ctypes.c_int))[0] == 2  # GGML_BACKEND_API_VERSION
    assert b.ggml_backend_init() == reg  # the entry point ggml_backend_load looks up
    ok = ctypes.CFUNCTYPE(ctypes.c_bool)(h.ggml_backend_reg_get_proc_address(reg, b"ggml_backend_mi355x_abi_ok"))
    assert ok()
    assert not h.ggml_backend_reg_get_proc_address(reg, b"no_such_function")


def test_a_ggml_with_other_op_numbers_gets_no_device():
    """A ggml from before ADD_ID (every later op numbered one lower): the registry logs the first difference and
    registers no device, rather than running MUL where that ggml asked for DIV, or MUL_MAT for MUL_MAT_ID."""
    skewed = ROOT / "tests" / "ggml_host" / "libggml_host_skewed.so"
    code = textwrap.dedent(f"""
        import ctypes, sys
        host = ctypes.CDLL({str(skewed)!r}, mode=ctypes.RTLD_GLOBAL)
        b = ctypes.CDLL({str(G.BACKEND_PATH)!r}, mode=ctypes.RTLD_GLOBAL)
        b.ggml_backend_mi355x_reg.restype = ctypes.c_void_p
        host.ggml_backend_reg_dev_count.restype = ctypes.c_size_t
        host.ggml_backend_reg_dev_count.argtypes = [ctypes.c_void_p]
        host.ggml_backend_reg_get_proc_address.restype = ctypes.c_void_p
        host.ggml_backend_reg_get_proc_address.argtypes = [ctypes.c_void_p, ctypes.c_char_p]
        host.ggml_host_last_log.restype = ctypes.c_char_p
        reg = b.ggml_backend_mi355x_reg()
        ok = ctypes.CFUNCTYPE(ctypes.c_bool)(host.ggml_backend_reg_get_proc_address(reg, b"ggml_backend_mi355x_abi_ok"))
        print(int(ok()), host.ggml_backend_reg_dev_count(reg), host.ggml_host_last_log().decode().strip())
    """)
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, check=True, timeout=120)
    ok, n, log = out.stdout.strip().split(" ", 2)
    assert ok == "0" and n == "0"
    assert "op 'DIV' where this backend was built with 'MUL'" in log


def expected_plan(n_layer, tail):
    per_layer = ["norm_products", "attention", "product_out", "norm_products", "product_out"]
    return ["node"] + per_layer * n_layer + tail


def test_plan_of_a_decode_step():
    """Qwen3Decoder::step's graph (Readback::Pick): per layer, the attention norm into q/k/v, the attention block as
    one step, attn_o + residual, the FFN norm into gate/up, SwiGLU + down + residual; then out_norm into the head."""
    st = G.Qwen3Step(2, 1024, 2048, 8, 4, 128, 1000, 256, 1, 128)
    try:
        assert [k for k, _ in G.plan(st.g)] == expected_plan(2, ["norm_products", "node"])
    finally:
        st.close()


def test_plan_keeps_what_the_graph_reads_back():
    """Readback::LogitsAndHidden marks the hidden state an output: its norm and weight run as their own nodes and the
    head as a plain product. A roped q marked an output keeps layer 0's attention block unfused. A block of four rows
    plans as one row does (its fused kernels decline at run time)."""
    st = G.Qwen3Step(2, 1024, 2048, 8, 4, 128, 1000, 256, 4, 128, readback="hidden", roped_q_output=True)
    try:
        kinds = [k for k, _ in G.plan(st.g)]
        assert kinds.count("attention") == 1
        assert kinds[-3:] == ["node", "node", "products"]
        assert kinds[2:11] == ["node"] * 9  # layer 0: q/k norms, v store, RoPEs, k store, attention
    finally:
        st.close()


def fake_addresses(tensors, alias=None):
    """Distinct, aligned data addresses for a graph's own tensors (views get their source's plus offset), as a
    placement without reuse would give them; alias = (a, b) puts b at a's address, as an allocator reusing a's memory
    for b would. The plan reads addresses only."""
    addr = 1 << 40
    for t in tensors:
        c = t.contents
        if not c.view_src:
            c.data = addr
            addr += (G.libs()[0].ggml_nbytes(t) + 255) // 256 * 256 + 256
    if alias:
        alias[1].contents.data = alias[0].contents.data
    for t in tensors:
        c = t.contents
        if c.view_src:
            c.data = ctypes.cast(c.view_src, ctypes.POINTER(G.Tensor)).contents.data + c.view_offs


def test_plan_of_a_moe_ffn():
    """TextModel::experts' gate and up MUL_MAT_IDs (same rows, same chosen experts) plan as one step at gate's place,
    the node between them after it; down stays a node. When up's output would reuse memory gate still holds for the
    node between them (an allocator reusing gate's memory after that node), the two run as their own nodes."""
    m = G.MoeFfn(2048, 1536, 64, 4, 16)
    try:
        fake_addresses(m.g.tensors)
        assert [k for k, _ in G.plan(m.g)] == ["experts", "node", "node", "node"]
        fake_addresses(m.g.tensors, alias=(m.gate, m.up))
        assert [k for k, _ in G.plan(m.g)] == ["node"] * 5
    finally:
        m.close()


def router_split_graph(H, E, T, n_used, later):
    """A Drama-3 FFN's front (text-model.cpp:198-221): the FFN norm x weight feeds the router product, and -- after the
    router's softmax and top-k, which stay on the CPU and split the scheduled graph there -- the routed experts read
    it again. Returns (graph, tensors by name, index of the first node of the second split)."""
    g = G.Graph()
    t = dict(x=g.new(G.F32, H, T), nw=g.new(G.F32, H), wr=g.new(G.Q8_0, H, E), ex=g.new(G.Q4_K, H, 256, E),
             sel=g.new(G.I32, n_used, T))
    t["h"] = g.mul(g.rms_norm(t["x"], 1e-6), t["nw"])
    t["r"] = g.mul_mat(t["wr"], t["h"])
    g.h.ggml_set_output(t["r"])
    g.expand(t["r"])
    if later:
        t["e"] = g.mul_mat_id(t["ex"], g.reshape_3d(t["h"], H, 1, T), t["sel"])
        g.h.ggml_set_output(t["e"])
        g.expand(t["e"])
    return g, t, g.index(t["r"]) + 1


def test_plan_of_a_split_keeps_what_a_later_split_reads():
    """Under ggml_backend_sched the backend computes one split of the graph at a time, a view sharing the whole graph's
    use counts. When a later split reads the norm x weight again, the split holding the router product keeps norm and
    weight as their own nodes (the fused product would not write them); with no later reader the same split fuses."""
    for later, want in ((True, ["node", "node", "products"]), (False, ["norm_products"])):
        g, t, cut = router_split_graph(2048, 8, 4, 4, later)
        try:
            v = g.view(0, cut)
            assert [k for k, _ in G.plan(v)] == want
        finally:
            g.close()


def test_plan_of_a_decode_split_with_readers_beyond_it():
    """A decode step whose intermediates a node after it reads (as a later split of a scheduled graph would): the
    product a fusion would leave unwritten (layer 0's down product before its residual ADD, layer 1's q/k/v group's
    norm x weight) is then computed as its own node in the step's split, counted over the whole graph; the other
    layers' fusions stay."""
    base = G.Qwen3Step(2, 1024, 2048, 8, 4, 128, 1000, 256, 1, 128)
    st = G.Qwen3Step(2, 1024, 2048, 8, 4, 128, 1000, 256, 1, 128)
    try:
        n = st.g.h.ggml_graph_n_nodes(st.g.graph)
        extra = st.g.add(st.taps[0]["dn"], st.taps[0]["dn"])  # a later reader of layer 0's down product
        extra2 = st.g.mul(st.taps[1]["h"], st.taps[1]["h"])  # and of layer 1's attention norm x weight
        st.g.h.ggml_set_output(extra)
        st.g.h.ggml_set_output(extra2)
        st.g.expand(extra)
        st.g.expand(extra2)
        assert st.g.h.ggml_graph_n_nodes(st.g.graph) == n + 2
        want = [k for k, _ in G.plan(base.g)]
        got = [k for k, _ in G.plan(st.g.view(0, n))]  # the step's own nodes, as one split
        assert want.count("product_out") == 4 and got.count("product_out") == 3
        assert want.count("norm_products") == 5 and got.count("norm_products") == 4
        assert got.count("attention") == want.count("attention") == 2
    finally:
        st.close()
        base.close()


# --------------------------------------------------------------------------------------------- on MI355X
@pytest.fixture(scope="module")
def device():
    d = G.Device()
    yield d
    d.close()


@pytest.mark.gpu
def test_device_through_the_registry(device):
    h = device.h
    assert h.ggml_backend_dev_type(device.dev) == 1  # GPU
    assert h.ggml_backend_dev_name(device.dev) == b"MI355X0"
    props = G.DevProps()
    h.ggml_backend_dev_get_props(device.dev, ctypes.byref(props))
    assert props.memory_total > 200 << 30 and 0 < props.memory_free <= props.memory_total
    assert props.caps.async_ and props.caps.events and not props.caps.host_buffer
    assert h.ggml_backend_buft_name(device.buft) == b"MI355X" and not h.ggml_backend_buft_is_host(device.buft)
    assert h.ggml_backend_dev_supports_buft(device.dev, device.buft)
    assert device.align == 256
    ev = h.ggml_backend_event_new(device.dev)
    h.ggml_backend_event_record(ev, device.backend)
    h.ggml_backend_event_synchronize(ev)
    h.ggml_backend_event_free(ev)


@pytest.mark.gpu
def test_buffer_transfers(device):
    """tensor_set in pieces at offsets inside blocks, get, memset, copy between device tensors, buffer clear."""
    g = G.Graph()
    try:
        K, N = 1024, 300
        w = O.quantize_chunk(O.TYPE_Q6_K, O.fill_normal(0x6B00, N, K, 0.0, 0.02))
        a, c = g.new(G.Q6_K, K, N), g.new(G.Q6_K, K, N)
        buf = device.place([a, c])
        device.upload(a, w, piece=1000)  # pieces that cut blocks and rows
        assert np.array_equal(device.download(a, np.uint8, w.shape), w)
        device.h.ggml_backend_tensor_copy(a, c)
        assert np.array_equal(device.download(c, np.uint8, w.shape), w)
        device.h.ggml_backend_tensor_memset(c, 0, 210 * 5, 210 * 3)  # three blocks of row 1
        got = device.download(c, np.uint8, w.shape).reshape(-1)
        ref = w.reshape(-1).copy()
        ref[210 * 5:210 * 8] = 0
        assert np.array_equal(got, ref)
        device.h.ggml_backend_buffer_clear(buf, 0)
        assert not device.download(a, np.uint8, w.shape).any()
    finally:
        g.close()


@pytest.mark.gpu
def test_copy_lands_before_the_next_compute(device):
    """ggml_backend_tensor_copy between two device tensors (ModelFile's copy, model-file.cpp:153-158), then at once a
    product reading the copy on the backend's own stream: the copy has landed when the call returns."""
    K, N, T = 4096, 16384, 2
    g = G.Graph()
    try:
        a, c = g.new(G.Q8_0, K, N), g.new(G.Q8_0, K, N)
        n0 = len(g.tensors)
        x = g.new(G.F32, K, T)
        y = g.mul_mat(c, x)
        g.h.ggml_set_output(y)
        g.expand(y)
        device.place([a, c], usage=1)
        device.place(g.tensors[n0:])
        w = O.quantize_chunk(O.TYPE_Q8_0, O.fill_normal(0x7C00, N, K, 0.0, 0.02))
        xv = O.fill_normal(0x7C01, T, K)
        device.upload(a, w)
        device.upload(x, xv)
        device.h.ggml_backend_tensor_memset(c, 0, 0, device.h.ggml_nbytes(c))
        device.h.ggml_backend_tensor_copy(a, c)
        device.compute(g)
        assert rel_err(device.download(y, np.float32, (T, N)), O.mul_mat(O.TYPE_Q8_0, w, xv)) <= TIGHT
    finally:
        g.close()


@pytest.mark.gpu
def test_scheduled_splits_keep_intermediates_and_replay(device):
    """A graph computed as two splits, as ggml_backend_sched computes Drama 3's (text-model.cpp:91-97): the first holds
    the FFN norm x weight and the router product, the second the routed experts reading that norm x weight again.
    The first split writes it (a later split reads it), and each split is recorded and replayed on its own: computed
    alternately four times, each is eager twice, recorded on its third computation and replayed on its fourth."""
    H, E, T, n_used = 2048, 8, 4, 4
    g, t, cut = router_split_graph(H, E, T, n_used, True)
    try:
        n = g.h.ggml_graph_n_nodes(g.graph)
        weights = [t["nw"], t["wr"], t["ex"]]
        device.place(weights, usage=1)
        device.place([u for u in g.tensors if all(ctypes.addressof(u.contents) != ctypes.addressof(w.contents)
                                                  for w in weights)])
        device.init_views(g.tensors)
        nw = O.fill_normal(0x7D00, 1, H, 1.0, 0.1)[0]
        wr = O.quantize_chunk(O.TYPE_Q8_0, O.fill_normal(0x7D01, E, H, 0.0, 0.02))
        ex = O.quantize_chunk(O.TYPE_Q4_K, O.fill_normal(0x7D02, E * 256, H, 0.0, 0.02))
        device.upload(t["nw"], nw)
        device.upload(t["wr"], wr)
        device.upload(t["ex"], ex)
        rng = np.random.default_rng(0x7D10)
        before = device.counters()
        for step in range(4):
            xv = O.fill_normal(int(rng.integers(1 << 30)), T, H)
            sel = np.stack([rng.choice(E, n_used, replace=False) for _ in range(T)]).astype(np.int32)
            device.upload(t["x"], xv)
            device.upload(t["sel"], sel)
            device.compute_split(g, 0, cut)
            device.compute_split(g, cut, n)
            h = O.binary("mul", O.rms_norm(xv, 1e-6), nw)
            assert rel_err(device.download(t["r"], np.float32, (T, E)), O.mul_mat(O.TYPE_Q8_0, wr, h)) <= TIGHT
            got = device.download(t["e"], np.float32, (T, n_used, 256))
            want = O.mul_mat_id(O.TYPE_Q4_K, ex.reshape(E, 256, -1), h.reshape(T, 1, H), sel)
            assert rel_err(got, want) <= TIGHT, f"step {step}"
        after = device.counters()
        assert [after[c] - before[c] for c in ("eager", "recorded", "replayed")] == [4, 2, 2]
    finally:
        g.close()


@pytest.mark.gpu
def test_products_graph_eager_record_replay(device):
    """GET_ROWS from a Q8_0 table of 17.4 MB (two upload pieces, the second starting inside a row), a q/k/v group of
    Q4_K products on its rows, MUL_MAT_ID over Q8_0 experts, a Q6_K head and ARGMAX, computed four times with new
    inputs: eagerly twice, recorded on the third, replayed on the fourth, each against the oracle."""
    H, V, E, Nx, n_used, T, Vh = 1024, 16000, 8, 128, 2, 3, 2000
    g = G.Graph()
    try:
        tab = g.new(G.Q8_0, H, V)
        wq, wk, wv = g.new(G.Q4_K, H, 512), g.new(G.Q4_K, H, 256), g.new(G.Q4_K, H, 256)
        ex = g.new(G.Q8_0, H, Nx, E)
        head = g.new(G.Q6_K, H, Vh)
        weights = [tab, wq, wk, wv, ex, head]
        n0 = len(g.tensors)
        ids = g.new(G.I32, T)
        sel = g.new(G.I32, n_used, T)
        emb = g.get_rows(tab, ids)
        q, k, v = g.mul_mat(wq, emb), g.mul_mat(wk, emb), g.mul_mat(wv, emb)
        moe = g.mul_mat_id(ex, g.reshape_3d(emb, H, 1, T), sel)
        logits = g.mul_mat(head, emb)
        pick = g.argmax(logits)
        for t in (q, k, v, moe, logits, pick):
            g.h.ggml_set_output(t)
            g.expand(t)
        data = {
            "tab": O.quantize_chunk(O.TYPE_Q8_0, O.fill_normal(0x7A00, V, H, 0.0, 0.5)),
            "wq": O.quantize_chunk(O.TYPE_Q4_K, O.fill_normal(0x7A01, 512, H, 0.0, 0.02)),
            "wk": O.quantize_chunk(O.TYPE_Q4_K, O.fill_normal(0x7A02, 256, H, 0.0, 0.02)),
            "wv": O.quantize_chunk(O.TYPE_Q4_K, O.fill_normal(0x7A03, 256, H, 0.0, 0.02)),
            "ex": O.quantize_chunk(O.TYPE_Q8_0, O.fill_normal(0x7A04, E * Nx, H, 0.0, 0.02)),
            "head": O.quantize_chunk(O.TYPE_Q6_K, O.fill_normal(0x7A05, Vh, H, 0.0, 0.02)),
        }
        device.place(weights, usage=1)
        device.place(g.tensors[n0:])
        device.init_views(g.tensors)
        for t, key in zip(weights, ["tab", "wq", "wk", "wv", "ex", "head"]):
            device.upload(t, data[key])
        for n in g.nodes():
            if n.contents.op != G.op_ids()["RESHAPE"]:
                assert device.supports(n), n.contents.op
        before = device.counters()
        rng = np.random.default_rng(0x7A10)
        for step in range(4):
            tok = rng.integers(0, V, T).astype(np.int32)
            tok[0] = V - 1
            choice = np.stack([rng.choice(E, n_used, replace=False) for _ in range(T)]).astype(np.int32)
            device.upload(ids, tok)
            device.upload(sel, choice)
            device.compute(g)
            x = O.get_rows(O.TYPE_Q8_0, data["tab"], H, tok)
            assert np.array_equal(device.download(emb, np.float32, (T, H)).view(np.uint32), x.view(np.uint32))
            for t, key, n in ((q, "wq", 512), (k, "wk", 256), (v, "wv", 256)):
                assert rel_err(device.download(t, np.float32, (T, n)), O.mul_mat(O.TYPE_Q4_K, data[key], x)) <= TIGHT
            y = O.mul_mat_id(O.TYPE_Q8_0, data["ex"].reshape(E, Nx, -1), x.reshape(T, 1, H), choice)
            assert rel_err(device.download(moe, np.float32, (T, n_used, Nx)), y) <= TIGHT
            lg = device.download(logits, np.float32, (T, Vh))
            assert rel_err(lg, O.mul_mat(O.TYPE_Q6_K, data["head"], x)) <= TIGHT
            assert np.array_equal(device.download(pick, np.int32, (T,)), O.argmax(lg)), f"step {step}"
        after = device.counters()
        assert [after[c] - before[c] for c in ("eager", "recorded", "replayed")] == [2, 1, 1]
    finally:
        g.close()


@pytest.mark.gpu
@pytest.mark.parametrize("T", [3, 24], ids=["matvec_path", "grouped"])
def test_moe_ffn_graph(device, T):
    """TextModel::experts' routed experts through graph_compute: gate and up in one MUL_MAT_ID group (one mat-vec
    launch for 6 pairs, the grouped Q4_K product for 48), the MULs around them, down over their product; each
    product against the oracle on the device's own inputs, twice (eager) with new routing. Then the same graph with
    up's output placed over gate's memory (valid for the graph's own order: gate is dead once the MUL has read it)
    runs gate and up as separate nodes, and still computes the right values."""
    H, F, E, n_used = 1024, 256, 8, 2
    m = G.MoeFfn(H, F, E, n_used, T)
    try:
        data = {k: O.quantize_chunk(O.TYPE_Q4_K, O.fill_normal(0x7B00 + i, n * E, kk, 0.0, 0.02))
                for i, (k, n, kk) in enumerate((("gate", F, H), ("up", F, H), ("down", H, F)))}
        device.place(m.weights, usage=1)
        for t, k in zip(m.weights, ("gate", "up", "down")):
            device.upload(t, data[k])
        rng = np.random.default_rng(0x7B10 + T)

        def run_and_check():
            x = O.fill_normal(int(rng.integers(1 << 30)), T, H)
            choice = np.stack([rng.choice(E, n_used, replace=False) for _ in range(T)]).astype(np.int32)
            device.upload(m.x, x)
            device.upload(m.sel, choice)
            device.compute(m.g)
            g2 = device.download(m.g2, np.float32, (T, n_used, F))
            up = device.download(m.up, np.float32, (T, n_used, F))
            gate = O.mul_mat_id(O.TYPE_Q4_K, data["gate"].reshape(E, F, -1), x.reshape(T, 1, H), choice)
            assert rel_err(g2, gate * gate) <= 4 * TIGHT
            assert rel_err(up, O.mul_mat_id(O.TYPE_Q4_K, data["up"].reshape(E, F, -1), x.reshape(T, 1, H), choice)) <= TIGHT
            act = g2 * up
            down = device.download(m.down, np.float32, (T, n_used, H))
            assert rel_err(down, O.mul_mat_id(O.TYPE_Q4_K, data["down"].reshape(E, H, -1), act, choice)) <= TIGHT

        device.place(m.compute)
        device.init_views(m.g.tensors)
        before = device.counters()
        for _ in range(2):
            run_and_check()
        after = device.counters()
        assert after["experts_group"] - before["experts_group"] == 2 and after["declined"] == before["declined"]

        # up over gate's memory: the planner must not run up ahead of the MUL that reads gate
        m.up.contents.data = m.gate.contents.data  # same buffer, same size: as an allocator reusing gate's memory
        before = device.counters()
        run_and_check()
        after = device.counters()
        assert after["experts_group"] == before["experts_group"]
    finally:
        m.close()


def oracle_step(st, data, caches, tok, past):
    """Qwen3Decoder::step in the oracle (attention in its exact form): the logits of one token; caches updated."""
    s = st.shape
    H, hd, nq, nkv, n_kv, eps, theta, t = s["H"], s["hd"], s["nq"], s["nkv"], s["n_kv"], s["eps"], s["theta"], s["wtype"]
    kv = nkv * hd
    pos = np.array([past], np.int32)
    mask = G.causal_mask(past, 1, n_kv)
    x = O.get_rows(t, data["head"], H, np.array([tok], np.int32))
    for l, d in enumerate(data["layers"]):
        h = O.binary("mul", O.rms_norm(x, eps), d["attn_norm"])
        q, k, v = (O.mul_mat(t, d[n], h) for n in ("wq", "wk", "wv"))
        q = O.rope_neox(O.binary("mul", O.rms_norm(q.reshape(1, nq, hd), eps), d["q_norm"]), pos, hd, theta)
        k = O.rope_neox(O.binary("mul", O.rms_norm(k.reshape(1, nkv, hd), eps), d["k_norm"]), pos, hd, theta)
        caches[l]["k"] = O.set_rows_f16(caches[l]["k"], k.reshape(1, kv), pos)
        caches[l]["v"] = O.set_rows_f16(caches[l]["v"], v.reshape(1, kv), pos)
        kc = caches[l]["k"][:n_kv].reshape(n_kv, nkv, hd).transpose(1, 0, 2)
        vc = caches[l]["v"][:n_kv].reshape(n_kv, nkv, hd).transpose(1, 0, 2)
        att = O.flash_attn_ext(q.transpose(1, 0, 2), kc, vc, mask, 1.0 / np.sqrt(hd), exact=True)
        x = O.binary("add", x, O.mul_mat(t, d["wo"], att.reshape(1, -1)))
        h = O.binary("mul", O.rms_norm(x, eps), d["ffn_norm"])
        x = O.binary("add", x, O.mul_mat(t, d["w_down"], O.swiglu(O.mul_mat(t, d["w_gate"], h),
                                                                  O.mul_mat(t, d["w_up"], h))))
    return O.mul_mat(t, data["head"], O.binary("mul", O.rms_norm(x, eps), data["out_norm"]))


@pytest.mark.gpu
def test_decode_graph_fused(device):
    """Two Qwen3 layers (hidden 1024, 8 q / 4 kv heads of 128, FFN 2048, Q8_0, f16 caches holding 70 positions)
    stepped four times through graph_compute as Qwen3Decoder::step builds the graph: eagerly twice, recorded, replayed,
    with the fused kernels (norm into q/k/v and gate/up, the attention block in one launch, SwiGLU + down + residual,
    attn_o + residual, out_norm into the head). Logits within 2e-4 of their largest value from the oracle's chain,
    the pick the first of the largest logits, the caches' new rows as the oracle stores them."""
    L, H, F, nq, nkv, hd, V, cap, past0 = 2, 1024, 2048, 8, 4, 128, 1000, 256, 70
    n_kv = 128  # round_up(past + 1, 64) for every step here
    st = G.Qwen3Step(L, H, F, nq, nkv, hd, V, cap, 1, n_kv)
    try:
        kv = nkv * hd
        t = O.TYPE_Q8_0
        qz = lambda seed, n, k: O.quantize_chunk(t, O.fill_normal(seed, n, k, 0.0, 0.05))
        vec = lambda seed, n: O.fill_normal(seed, 1, n, 1.0, 0.1)[0]
        data = {"head": O.quantize_chunk(t, O.fill_normal(0x7B00, V, H, 0.0, 0.5)), "out_norm": vec(0x7B01, H),
                "layers": []}
        caches = []
        for l in range(L):
            b = 0x7C00 + 32 * l
            data["layers"].append(dict(
                attn_norm=vec(b, H), wq=qz(b + 1, nq * hd, H), wk=qz(b + 2, kv, H), wv=qz(b + 3, kv, H),
                q_norm=vec(b + 4, hd), k_norm=vec(b + 5, hd), wo=qz(b + 6, H, nq * hd), ffn_norm=vec(b + 7, H),
                w_gate=qz(b + 8, F, H), w_up=qz(b + 9, F, H), w_down=qz(b + 10, H, F)))
            c = {}
            for j, n in enumerate(("k", "v")):
                c[n] = np.zeros((cap, kv), np.uint16)
                c[n][:past0] = O.fill_normal(b + 11 + j, past0, kv).astype(np.float16).view(np.uint16)
            caches.append(c)
        device.place(st.weights, usage=1)
        device.place(st.compute)
        device.init_views(st.g.tensors)
        device.upload(st.head, data["head"])
        device.upload(st.out_norm, data["out_norm"])
        for d, w, c in zip(st.layers, data["layers"], caches):
            for name, arr in w.items():
                device.upload(d[name], arr)
            device.upload(d["kc"], c["k"])
            device.upload(d["vc"], c["v"])
        for n in st.g.nodes():
            if n.contents.op not in [G.op_ids()[o] for o in ("RESHAPE", "VIEW", "PERMUTE")]:
                assert device.supports(n), n.contents.op
        before = device.counters()
        tok = 17
        for step in range(4):
            past = past0 + step
            device.upload(st.tok, np.array([tok], np.int32))
            device.upload(st.pos, np.array([past], np.int32))
            device.upload(st.mask, G.causal_mask(past, 1, n_kv))
            device.compute(st.g)
            ref = oracle_step(st, data, caches, tok, past)
            got = device.download(st.logits, np.float32, (1, V))
            assert np.abs(got - ref).max() <= 2e-4 * np.abs(ref).max(), f"step {step}"
            pick = int(device.download(st.pick, np.int32, (1,))[0])
            assert pick == int(O.argmax(got)[0])
            for d, c in zip(st.layers, caches):
                for n in ("k", "v"):
                    row = device.download(d[n + "c"], np.uint16, (cap, kv))[past]
                    assert np.abs(row.view(np.float16).astype(np.float32) -
                                  c[n][past].view(np.float16).astype(np.float32)).max() <= 2e-3, (step, n)
            tok = pick
        after = device.counters()
        diff = {c: after[c] - before[c] for c in after}
        assert (diff["eager"], diff["recorded"], diff["replayed"]) == (2, 1, 1)
        # three graphs run node by node (two eager, one recorded): per graph 2 attention blocks, 2 * 2 + 1 norms
        # into products, 2 * 2 products with a residual, nothing declined
        assert (diff["attention"], diff["norm_products"], diff["product_out"], diff["declined"]) == (6, 15, 12, 0)
    finally:
        st.close()


def check_gemm(t, w, x, y):
    """A prefill product as the dispatcher runs it: Q8_0 at K % 128 == 0 on the int8 GEMM, which sums the oracle's
    exact per-block integers (held to TIGHT); otherwise on the fp16 dequantizing GEMM, against what it computes (the
    dq model, up to fp32 summation order) and against the oracle within the products' 1e-3 bar."""
    if t == O.TYPE_Q8_0 and x.shape[1] % 128 == 0:
        assert rel_err(y, O.mul_mat(t, w, x)) <= TIGHT
        return
    assert rel_err(y, dq_model(O, t, w, x, x.shape[1])) <= TIGHT
    assert rel_err(y, O.mul_mat(t, w, x)) <= 1e-3


@pytest.mark.gpu
def test_prefill_graph_declines_to_separate_ops(device):
    """Twelve rows at once (a prefill block, Qwen3Decoder::run): the fused mat-vec kernels take at most 8 columns, so
    the norm and residual fusions run as their separate nodes (the products on the GEMMs) and the attention block's
    norms, RoPE and stores fuse in their rows form. Every node the graph writes is held to the oracle applied to the
    device's own inputs of that node, at the bar of the op's own tests: GET_ROWS, ADD and the cache rows of v
    bit-exact, norms within 2 float ulps, RoPE and SwiGLU within 1e-5, attention within 1e-5 of a row's largest
    output, products as check_gemm. The chain as a whole is held loosely to the exact oracle chain (2e-2 of the
    largest value): fp16 rounding of q in the attention and Q8_0 rounding of activations are discontinuous, and the
    FFN magnifies a code that a last-bit difference moves (the oracle chain with products computed the GEMM's way is
    itself 1.1e-2 of the largest hidden value from the exact chain)."""
    L, H, F, nq, nkv, hd, V, cap, past, rows = 1, 1024, 2048, 8, 4, 128, 500, 256, 30, 12
    n_kv = 64
    st = G.Qwen3Step(L, H, F, nq, nkv, hd, V, cap, rows, n_kv, readback="hidden")
    try:
        kv = nkv * hd
        t = O.TYPE_Q8_0
        qz = lambda seed, n, k: O.quantize_chunk(t, O.fill_normal(seed, n, k, 0.0, 0.05))
        vec = lambda seed, n: O.fill_normal(seed, 1, n, 1.0, 0.1)[0]
        head = O.quantize_chunk(t, O.fill_normal(0x7D00, V, H, 0.0, 0.5))
        out_norm = vec(0x7D01, H)
        w = dict(attn_norm=vec(0x7D02, H), wq=qz(0x7D03, nq * hd, H), wk=qz(0x7D04, kv, H), wv=qz(0x7D05, kv, H),
                 q_norm=vec(0x7D06, hd), k_norm=vec(0x7D07, hd), wo=qz(0x7D08, H, nq * hd), ffn_norm=vec(0x7D09, H),
                 w_gate=qz(0x7D0A, F, H), w_up=qz(0x7D0B, F, H), w_down=qz(0x7D0C, H, F))
        cache = {n: np.zeros((cap, kv), np.uint16) for n in ("k", "v")}
        for j, n in enumerate(("k", "v")):
            cache[n][:past] = O.fill_normal(0x7D10 + j, past, kv).astype(np.float16).view(np.uint16)
        device.place(st.weights, usage=1)
        device.place(st.compute)
        device.init_views(st.g.tensors)
        device.upload(st.head, head)
        device.upload(st.out_norm, out_norm)
        d = st.layers[0]
        for name, arr in w.items():
            device.upload(d[name], arr)
        device.upload(d["kc"], cache["k"])
        device.upload(d["vc"], cache["v"])
        toks = np.array([5, 77, 123, 499, 0, 1, 2, 250, 251, 17, 17, 300], np.int32)
        pos = np.arange(past, past + rows, dtype=np.int32)
        mask = G.causal_mask(past, rows, n_kv)
        device.upload(st.tok, toks)
        device.upload(st.pos, pos)
        device.upload(st.mask, mask)
        before = device.counters()
        device.compute(st.g)
        after = device.counters()
        diff = {c: after[c] - before[c] for c in after}
        assert diff["attention_rows"] == 1 and diff["attention"] == 0 and diff["declined"] == 4
        eps, theta, scale = 1e-6, 1e6, 1.0 / np.sqrt(hd)
        tap, d = st.taps[0], st.layers[0]
        f = lambda name, n: device.download(tap[name], np.float32, (rows, n))
        x = f("x", H)
        assert np.array_equal(x.view(np.uint32), O.get_rows(t, head, H, toks).view(np.uint32))
        h = f("h", H)
        assert ulps(h, O.binary("mul", O.rms_norm(x, eps), w["attn_norm"])) <= 2
        q, k, v = f("q", nq * hd), f("k", kv), f("v", kv)
        for y, name in ((q, "wq"), (k, "wk"), (v, "wv")):
            check_gemm(t, w[name], h, y)
        qr = device.download(tap["qr"], np.float32, (rows, nq, hd))
        qr_ref = O.rope_neox(O.binary("mul", O.rms_norm(q.reshape(rows, nq, hd), eps), w["q_norm"]), pos, hd, theta)
        assert np.abs(qr - qr_ref).max() <= 1e-5 * np.abs(qr_ref).max()
        kr_ref = O.rope_neox(O.binary("mul", O.rms_norm(k.reshape(rows, nkv, hd), eps), w["k_norm"]), pos, hd, theta)
        kc = device.download(d["kc"], np.uint16, (cap, kv))
        vc = device.download(d["vc"], np.uint16, (cap, kv))
        assert np.array_equal(vc, O.set_rows_f16(cache["v"], v, pos))
        k_new = kc[past:past + rows].view(np.float16).astype(np.float32)
        k_ref = O.set_rows_f16(cache["k"], kr_ref.reshape(rows, kv), pos)[past:past + rows]
        assert np.array_equal(kc[:past], cache["k"][:past])
        assert np.all(np.abs(k_new - k_ref.view(np.float16).astype(np.float32)) <= 2.0 ** -10 * np.abs(k_new) + 1e-7)
        att = f("att", nq * hd)
        att_ref = O.flash_attn_ext(qr.transpose(1, 0, 2), kc[:n_kv].reshape(n_kv, nkv, hd).transpose(1, 0, 2),
                                   vc[:n_kv].reshape(n_kv, nkv, hd).transpose(1, 0, 2), mask, scale, exact=True)
        att_ref = att_ref.reshape(rows, -1)
        assert (np.abs(att - att_ref).max(axis=1) / np.abs(att_ref).max(axis=1)).max() <= 1e-5
        ao = f("ao", H)
        check_gemm(t, w["wo"], att, ao)
        x1 = f("x1", H)
        assert np.array_equal(x1, O.binary("add", x, ao))
        h1 = f("h1", H)
        assert ulps(h1, O.binary("mul", O.rms_norm(x1, eps), w["ffn_norm"])) <= 2
        gate, up = f("gate", F), f("up", F)
        check_gemm(t, w["w_gate"], h1, gate)
        check_gemm(t, w["w_up"], h1, up)
        glu = f("glu", F)
        assert np.abs(glu - O.swiglu(gate, up)).max() <= 1e-5 * np.abs(glu).max()
        dn = f("dn", H)
        check_gemm(t, w["w_down"], glu, dn)
        x2 = f("x2", H)
        assert np.array_equal(x2, O.binary("add", x1, dn))
        hidden = device.download(st.hidden, np.float32, (rows, H))
        assert ulps(hidden, O.binary("mul", O.rms_norm(x2, eps), out_norm)) <= 2
        logits = device.download(st.logits, np.float32, (rows, V))
        check_gemm(t, head, hidden, logits)

        # the chain against the exact oracle chain
        xe = O.get_rows(t, head, H, toks)
        he = O.binary("mul", O.rms_norm(xe, eps), w["attn_norm"])
        qe, ke, ve = (O.mul_mat(t, w[n], he) for n in ("wq", "wk", "wv"))
        qe = O.rope_neox(O.binary("mul", O.rms_norm(qe.reshape(rows, nq, hd), eps), w["q_norm"]), pos, hd, theta)
        ke = O.rope_neox(O.binary("mul", O.rms_norm(ke.reshape(rows, nkv, hd), eps), w["k_norm"]), pos, hd, theta)
        kce = O.set_rows_f16(cache["k"], ke.reshape(rows, kv), pos)[:n_kv].reshape(n_kv, nkv, hd).transpose(1, 0, 2)
        vce = O.set_rows_f16(cache["v"], ve.reshape(rows, kv), pos)[:n_kv].reshape(n_kv, nkv, hd).transpose(1, 0, 2)
        ae = O.flash_attn_ext(qe.transpose(1, 0, 2), kce, vce, mask, scale, exact=True)
        xe = O.binary("add", xe, O.mul_mat(t, w["wo"], ae.reshape(rows, -1)))
        he = O.binary("mul", O.rms_norm(xe, eps), w["ffn_norm"])
        xe = O.binary("add", xe, O.mul_mat(t, w["w_down"], O.swiglu(O.mul_mat(t, w["w_gate"], he),
                                                                    O.mul_mat(t, w["w_up"], he))))
        hidden_e = O.binary("mul", O.rms_norm(xe, eps), out_norm)
        assert np.abs(hidden - hidden_e).max() <= 2e-2 * np.abs(hidden_e).max()
    finally:
        st.close()
