"""ctypes access to ggml's C API as the test host provides it (tests/ggml_host/libggml_host.so) and to the MI355X ggml
backend (speech.cpp_amd/libggml-mi355x.so) loaded beside it, so that tests drive the backend the way speech.cpp
does: registry -> device -> buffer type -> weight and compute buffers -> tensors placed, uploaded in 16 MB pieces
(src/common/model-file.cpp:222-268) -> graphs built with ggml's op constructors in Qwen3Decoder's order
(src/common/qwen3-decoder.cpp:350-438) -> ggml_backend_graph_compute (src/common/graph.cpp:96-110)."""
import ctypes
import pathlib

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[1]
HOST_PATH = ROOT / "tests" / "ggml_host" / "libggml_host.so"
BACKEND_PATH = ROOT / "speech.cpp_amd" / "libggml-mi355x.so"

F32, F16, Q8_0, Q4_K, Q5_K, Q6_K, I32 = 0, 1, 8, 12, 13, 14, 26
ROPE_NEOX = 2
FLAG_OUTPUT = 2
PIECE = 16 << 20  # the upload piece of model-file.cpp


class Tensor(ctypes.Structure):
    _fields_ = [("type", ctypes.c_int), ("buffer", ctypes.c_void_p), ("ne", ctypes.c_int64 * 4),
                ("nb", ctypes.c_size_t * 4), ("op", ctypes.c_int), ("op_params", ctypes.c_int32 * 16),
                ("flags", ctypes.c_int32), ("src", ctypes.c_void_p * 10), ("view_src", ctypes.c_void_p),
                ("view_offs", ctypes.c_size_t), ("data", ctypes.c_void_p), ("name", ctypes.c_char * 64),
                ("extra", ctypes.c_void_p), ("padding", ctypes.c_char * 8)]


class HashSet(ctypes.Structure):
    _fields_ = [("size", ctypes.c_size_t), ("used", ctypes.c_void_p), ("keys", ctypes.c_void_p)]


class CGraph(ctypes.Structure):
    """ggml_cgraph as ggml-impl.h lays it out (a view of a graph is one by value)."""
    _fields_ = [("size", ctypes.c_int), ("n_nodes", ctypes.c_int), ("n_leafs", ctypes.c_int),
                ("nodes", ctypes.c_void_p), ("grads", ctypes.c_void_p), ("grad_accs", ctypes.c_void_p),
                ("leafs", ctypes.c_void_p), ("use_counts", ctypes.c_void_p), ("visited_hash_set", HashSet),
                ("order", ctypes.c_int)]


class InitParams(ctypes.Structure):
    _fields_ = [("mem_size", ctypes.c_size_t), ("mem_buffer", ctypes.c_void_p), ("no_alloc", ctypes.c_bool)]


class DevCaps(ctypes.Structure):
    _fields_ = [("async_", ctypes.c_bool), ("host_buffer", ctypes.c_bool), ("buffer_from_host_ptr", ctypes.c_bool),
                ("events", ctypes.c_bool)]


class DevProps(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("description", ctypes.c_char_p), ("memory_free", ctypes.c_size_t),
                ("memory_total", ctypes.c_size_t), ("type", ctypes.c_int), ("device_id", ctypes.c_char_p),
                ("caps", DevCaps)]


TP = ctypes.POINTER(Tensor)
VP = ctypes.c_void_p
SZ = ctypes.c_size_t
I64 = ctypes.c_int64
FL = ctypes.c_float
INT = ctypes.c_int

_SIGS = {
    # core
    "ggml_init": (VP, [InitParams]), "ggml_free": (None, [VP]),
    "ggml_new_tensor_1d": (TP, [VP, INT, I64]), "ggml_new_tensor_2d": (TP, [VP, INT, I64, I64]),
    "ggml_new_tensor_3d": (TP, [VP, INT, I64, I64, I64]), "ggml_set_name": (TP, [TP, ctypes.c_char_p]),
    "ggml_set_output": (None, [TP]), "ggml_set_input": (None, [TP]), "ggml_nbytes": (SZ, [TP]),
    "ggml_row_size": (SZ, [INT, I64]), "ggml_op_name": (ctypes.c_char_p, [INT]),
    "ggml_add": (TP, [VP, TP, TP]), "ggml_mul": (TP, [VP, TP, TP]), "ggml_argmax": (TP, [VP, TP]),
    "ggml_rms_norm": (TP, [VP, TP, FL]), "ggml_mul_mat": (TP, [VP, TP, TP]),
    "ggml_mul_mat_id": (TP, [VP, TP, TP, TP]), "ggml_reshape_2d": (TP, [VP, TP, I64, I64]),
    "ggml_reshape_3d": (TP, [VP, TP, I64, I64, I64]),
    "ggml_view_3d": (TP, [VP, TP, I64, I64, I64, SZ, SZ, SZ]), "ggml_permute": (TP, [VP, TP, INT, INT, INT, INT]),
    "ggml_get_rows": (TP, [VP, TP, TP]), "ggml_set_rows": (TP, [VP, TP, TP, TP]),
    "ggml_rope_ext": (TP, [VP, TP, TP, TP, INT, INT, INT, FL, FL, FL, FL, FL, FL]),
    "ggml_flash_attn_ext": (TP, [VP, TP, TP, TP, TP, FL, FL, FL]), "ggml_flash_attn_ext_set_prec": (None, [TP, INT]),
    "ggml_swiglu_split": (TP, [VP, TP, TP]),
    "ggml_new_graph": (VP, [VP]), "ggml_build_forward_expand": (None, [VP, TP]),
    "ggml_graph_view": (CGraph, [VP, INT, INT]),
    "ggml_graph_n_nodes": (INT, [VP]), "ggml_graph_node": (TP, [VP, INT]),
    "ggml_host_last_log": (ctypes.c_char_p, []), "ggml_host_clear_log": (None, []),
    # backend
    "ggml_backend_reg_name": (ctypes.c_char_p, [VP]), "ggml_backend_reg_dev_count": (SZ, [VP]),
    "ggml_backend_reg_dev_get": (VP, [VP, SZ]), "ggml_backend_reg_get_proc_address": (VP, [VP, ctypes.c_char_p]),
    "ggml_backend_dev_name": (ctypes.c_char_p, [VP]), "ggml_backend_dev_description": (ctypes.c_char_p, [VP]),
    "ggml_backend_dev_type": (INT, [VP]), "ggml_backend_dev_get_props": (None, [VP, ctypes.POINTER(DevProps)]),
    "ggml_backend_dev_init": (VP, [VP, ctypes.c_char_p]), "ggml_backend_dev_buffer_type": (VP, [VP]),
    "ggml_backend_dev_supports_op": (ctypes.c_bool, [VP, TP]),
    "ggml_backend_dev_supports_buft": (ctypes.c_bool, [VP, VP]),
    "ggml_backend_buft_name": (ctypes.c_char_p, [VP]), "ggml_backend_buft_alloc_buffer": (VP, [VP, SZ]),
    "ggml_backend_buft_get_alignment": (SZ, [VP]), "ggml_backend_buft_get_alloc_size": (SZ, [VP, TP]),
    "ggml_backend_buft_is_host": (ctypes.c_bool, [VP]),
    "ggml_backend_buffer_free": (None, [VP]), "ggml_backend_buffer_get_base": (VP, [VP]),
    "ggml_backend_buffer_get_size": (SZ, [VP]), "ggml_backend_buffer_set_usage": (None, [VP, INT]),
    "ggml_backend_buffer_clear": (None, [VP, ctypes.c_uint8]),
    "ggml_backend_tensor_alloc": (INT, [VP, TP, VP]), "ggml_backend_view_init": (INT, [TP]),
    "ggml_backend_tensor_set": (None, [TP, VP, SZ, SZ]), "ggml_backend_tensor_get": (None, [TP, VP, SZ, SZ]),
    "ggml_backend_tensor_memset": (None, [TP, ctypes.c_uint8, SZ, SZ]),
    "ggml_backend_tensor_copy": (None, [TP, TP]),
    "ggml_backend_name": (ctypes.c_char_p, [VP]), "ggml_backend_free": (None, [VP]),
    "ggml_backend_synchronize": (None, [VP]), "ggml_backend_graph_compute": (INT, [VP, VP]),
    "ggml_host_graph_compute_split": (INT, [VP, VP, INT, INT]),
    "ggml_backend_supports_op": (ctypes.c_bool, [VP, TP]),
    "ggml_backend_event_new": (VP, [VP]), "ggml_backend_event_free": (None, [VP]),
    "ggml_backend_event_record": (None, [VP, VP]), "ggml_backend_event_synchronize": (None, [VP]),
}

COUNTERS = ["eager", "recorded", "replayed", "norm_products", "product_out", "attention", "attention_rows",
            "declined", "experts_group"]

_lib = None


def libs():
    """(host, backend): the host loaded first with its symbols global, so the backend's ggml references bind to it."""
    global _lib
    if _lib is None:
        for p in (HOST_PATH, BACKEND_PATH):
            if not p.exists():
                raise RuntimeError(f"{p} is not built (run __graft_entry__.build())")
        host = ctypes.CDLL(str(HOST_PATH), mode=ctypes.RTLD_GLOBAL)
        for name, (res, args) in _SIGS.items():
            f = getattr(host, name)
            f.restype, f.argtypes = res, args
        backend = ctypes.CDLL(str(BACKEND_PATH), mode=ctypes.RTLD_GLOBAL)
        backend.ggml_backend_mi355x_reg.restype = VP
        backend.ggml_backend_mi355x_reg.argtypes = []
        backend.ggml_backend_init.restype = VP
        backend.ggml_backend_init.argtypes = []
        _lib = (host, backend)
    return _lib


def op_ids():
    h, _ = libs()
    ids, i = {}, 0
    while True:
        n = h.ggml_op_name(i)
        if n is None:
            return ids
        ids[n.decode()] = i
        i += 1


class Graph:
    """One ggml context: tensors made through ggml's constructors, kept in creation order for placement."""

    def __init__(self):
        self.h, _ = libs()
        self.ctx = self.h.ggml_init(InitParams(0, None, True))
        self.tensors = []
        self.graph = self.h.ggml_new_graph(self.ctx)

    def close(self):
        if self.ctx:
            self.h.ggml_free(self.ctx)
            self.ctx = None

    def __getattr__(self, name):  # ggml_<op>(ctx, ...) as self.<op>(...)
        f = getattr(self.h, "ggml_" + name)

        def call(*args):
            t = f(self.ctx, *args)
            self.tensors.append(t)
            return t
        return call

    def new(self, t, *ne, name=None):
        fn = {1: self.h.ggml_new_tensor_1d, 2: self.h.ggml_new_tensor_2d, 3: self.h.ggml_new_tensor_3d}[len(ne)]
        x = fn(self.ctx, t, *ne)
        if name:
            self.h.ggml_set_name(x, name.encode())
        self.tensors.append(x)
        return x

    def expand(self, t):
        self.h.ggml_build_forward_expand(self.graph, t)

    def nodes(self):
        return [self.h.ggml_graph_node(self.graph, i) for i in range(self.h.ggml_graph_n_nodes(self.graph))]

    def index(self, t):
        """The position of node t in the graph."""
        addrs = [ctypes.addressof(n.contents) for n in self.nodes()]
        return addrs.index(ctypes.addressof(t.contents))

    def view(self, i0, i1):
        """Nodes [i0, i1) as ggml_backend_sched hands a backend one split: a view sharing the graph's use counts.
        Returns the view (a CGraph, kept by the caller while used)."""
        return self.h.ggml_graph_view(self.graph, i0, i1)


class Device:
    """The MI355X backend's first device, one backend (stream) on it, and its buffer type."""

    def __init__(self):
        self.h, self.b = libs()
        self.reg = self.b.ggml_backend_mi355x_reg()
        if self.h.ggml_backend_reg_dev_count(self.reg) < 1:
            raise RuntimeError("the MI355X backend registered no device")
        self.dev = self.h.ggml_backend_reg_dev_get(self.reg, 0)
        self.backend = self.h.ggml_backend_dev_init(self.dev, None)
        assert self.backend, self.h.ggml_host_last_log()
        self.buft = self.h.ggml_backend_dev_buffer_type(self.dev)
        self.align = self.h.ggml_backend_buft_get_alignment(self.buft)
        self.buffers = []
        fp = self.h.ggml_backend_reg_get_proc_address(self.reg, b"ggml_backend_mi355x_counters")
        self._counters = ctypes.CFUNCTYPE(None, VP, ctypes.POINTER(I64), INT)(fp)

    def close(self):
        for b in self.buffers:
            self.h.ggml_backend_buffer_free(b)
        self.buffers = []
        if self.backend:
            self.h.ggml_backend_free(self.backend)
            self.backend = None

    def counters(self):
        out = (I64 * len(COUNTERS))()
        self._counters(self.backend, out, len(COUNTERS))
        return dict(zip(COUNTERS, list(out)))

    def place(self, tensors, usage=0):
        """Allocates one buffer of this device's type for the tensors that own memory and places them in order at
        the buffer type's alignment (what ggml_backend_alloc_ctx_tensors / ggml_gallocr do without reuse); views are
        initialised over their sources afterwards."""
        own = [t for t in tensors if not t.contents.view_src and not t.contents.data]
        sizes = [self.h.ggml_backend_buft_get_alloc_size(self.buft, t) for t in own]
        offs, total = [], 0
        for s in sizes:
            total = (total + self.align - 1) // self.align * self.align
            offs.append(total)
            total += s
        buf = self.h.ggml_backend_buft_alloc_buffer(self.buft, max(total, 1))
        assert buf, self.h.ggml_host_last_log()
        self.buffers.append(buf)
        self.h.ggml_backend_buffer_set_usage(buf, usage)
        base = self.h.ggml_backend_buffer_get_base(buf)
        for t, o in zip(own, offs):
            assert self.h.ggml_backend_tensor_alloc(buf, t, base + o) == 0, self.h.ggml_host_last_log()
        return buf

    def init_views(self, tensors):
        for t in tensors:
            if t.contents.view_src and not t.contents.buffer:
                assert self.h.ggml_backend_view_init(t) == 0, self.h.ggml_host_last_log()

    def upload(self, t, arr, piece=PIECE):
        """ggml_backend_tensor_set in pieces, as model-file.cpp streams a weight (the last piece ragged)."""
        raw = np.ascontiguousarray(arr).reshape(-1).view(np.uint8)
        n = self.h.ggml_nbytes(t)
        assert raw.size == n, (raw.size, n)
        for off in range(0, n, piece):
            m = min(piece, n - off)
            self.h.ggml_backend_tensor_set(t, raw.ctypes.data + off, off, m)

    def download(self, t, dtype, shape):
        n = self.h.ggml_nbytes(t)
        out = np.empty(n, np.uint8)
        self.h.ggml_backend_tensor_get(t, out.ctypes.data, 0, n)
        return out.view(dtype).reshape(shape)

    def compute(self, g):
        st = self.h.ggml_backend_graph_compute(self.backend, g.graph)
        assert st == 0, (st, self.h.ggml_host_last_log())

    def compute_split(self, g, i0, i1):
        """Nodes [i0, i1) of g computed as one split of a scheduled graph."""
        st = self.h.ggml_host_graph_compute_split(self.backend, g.graph, i0, i1)
        assert st == 0, (st, self.h.ggml_host_last_log())

    def supports(self, t):
        return self.h.ggml_backend_dev_supports_op(self.dev, t)


STEPS = ["node", "products", "norm_products", "product_out", "attention", "experts"]


def plan(g):
    """The MI355X backend's plan of a graph (no device needed): [(step kind, index of its first node)]. g: a Graph, or
    a CGraph view of one (one split)."""
    h, b = libs()
    reg = b.ggml_backend_mi355x_reg()
    fp = h.ggml_backend_reg_get_proc_address(reg, b"ggml_backend_mi355x_plan")
    f = ctypes.CFUNCTYPE(INT, VP, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32), INT)(fp)
    kinds, first = (ctypes.c_int32 * 8192)(), (ctypes.c_int32 * 8192)()
    graph = ctypes.addressof(g) if isinstance(g, CGraph) else g.graph
    n = f(graph, kinds, first, 8192)
    return [(STEPS[kinds[i]], first[i]) for i in range(n)]


class MoeFfn:
    """The routed experts of a Drama-3 MoE FFN as TextModel::experts builds them (text-model.cpp:207-210): gate and up
    MUL_MAT_IDs over the same rows and chosen experts, then down over mul(silu(gate), up). Between gate and up sits a
    node that reads gate (ggml's order puts silu(gate) there); MUL nodes, which this backend computes, stand in for
    the silu: down reads (gate * gate) * up. Weights go in `weights`, the inputs and results in `compute`."""

    def __init__(self, H, F, E, n_used, T, wtype=Q4_K):
        g = self.g = Graph()
        self.shape = dict(H=H, F=F, E=E, n_used=n_used, T=T, wtype=wtype)
        self.gate_e, self.up_e, self.down_e = g.new(wtype, H, F, E), g.new(wtype, H, F, E), g.new(wtype, F, H, E)
        self.weights = [self.gate_e, self.up_e, self.down_e]
        n0 = len(g.tensors)
        self.x = g.new(F32, H, T)
        self.sel = g.new(I32, n_used, T)
        rows = g.reshape_3d(self.x, H, 1, T)
        self.gate = g.mul_mat_id(self.gate_e, rows, self.sel)
        self.g2 = g.mul(self.gate, self.gate)
        self.up = g.mul_mat_id(self.up_e, rows, self.sel)
        self.act = g.mul(self.g2, self.up)
        self.down = g.mul_mat_id(self.down_e, self.act, self.sel)
        for t in (self.g2, self.up, self.down):
            g.h.ggml_set_output(t)
        g.expand(self.down)
        self.compute = g.tensors[n0:]

    def close(self):
        self.g.close()


class Qwen3Step:
    """A Qwen3 decoder's graph for `rows` new tokens with flash attention, built as Qwen3Decoder builds it: GET_ROWS of
    the tokens from the tied embedding (qwen3-decoder.cpp:462-490), ::layers (:350-410) with its g.expand order, and
    ::outputs (:422-438) -- the greedy pick (Readback::Pick) or the logits and hidden state (LogitsAndHidden). Weights
    and the two f16 caches per layer go in `weights`, the inputs and everything computed in `compute`."""

    def __init__(self, n_layer, H, F, nq, nkv, hd, V, cap, rows, n_kv, eps=1e-6, theta=1e6, wtype=Q8_0,
                 readback="pick", roped_q_output=False):
        g = self.g = Graph()
        kv = nkv * hd
        self.shape = dict(n_layer=n_layer, H=H, F=F, nq=nq, nkv=nkv, hd=hd, V=V, cap=cap, rows=rows, n_kv=n_kv,
                          eps=eps, theta=theta, wtype=wtype)
        self.weights = []

        def W(t, *ne):
            x = g.new(t, *ne)
            self.weights.append(x)
            return x

        self.head = W(wtype, H, V)  # tied token embedding and output head
        self.layers = []
        for _ in range(n_layer):
            self.layers.append(dict(attn_norm=W(F32, H), wq=W(wtype, H, nq * hd), wk=W(wtype, H, kv),
                                    wv=W(wtype, H, kv), q_norm=W(F32, hd), k_norm=W(F32, hd), wo=W(wtype, nq * hd, H),
                                    ffn_norm=W(F32, H), w_gate=W(wtype, H, F), w_up=W(wtype, H, F),
                                    w_down=W(wtype, F, H), kc=W(F16, kv, cap), vc=W(F16, kv, cap)))
        self.out_norm = W(F32, H)
        n0 = len(g.tensors)
        self.tok = g.new(I32, rows)
        self.pos = g.new(I32, rows)
        self.mask = g.new(F16, n_kv, rows)
        x = self.emb = g.get_rows(self.head, self.tok)
        scale = 1.0 / np.sqrt(hd)
        self.taps = []  # per layer, the tensors each node writes (a fused step skips some of them)
        for li, d in enumerate(self.layers):
            tap = {"x": x}
            self.taps.append(tap)
            h = tap["h"] = g.mul(g.rms_norm(x, eps), d["attn_norm"])
            q, k, v = g.mul_mat(d["wq"], h), g.mul_mat(d["wk"], h), g.mul_mat(d["wv"], h)
            tap.update(q=q, k=k, v=v)
            g.expand(q)
            g.expand(k)
            g.expand(v)
            q = g.mul(g.rms_norm(g.reshape_3d(q, hd, nq, rows), eps), d["q_norm"])
            k = g.mul(g.rms_norm(g.reshape_3d(k, hd, nkv, rows), eps), d["k_norm"])
            g.expand(q)
            g.expand(k)
            g.expand(g.set_rows(d["vc"], v, self.pos))
            q = tap["qr"] = g.rope_ext(q, self.pos, None, hd, ROPE_NEOX, 0, theta, 1.0, 0.0, 1.0, 0.0, 0.0)
            k = g.rope_ext(k, self.pos, None, hd, ROPE_NEOX, 0, theta, 1.0, 0.0, 1.0, 0.0, 0.0)
            if roped_q_output and li == 0:
                g.h.ggml_set_output(q)
            g.expand(q)
            g.expand(g.set_rows(d["kc"], g.reshape_2d(k, kv, rows), self.pos))
            kc, vc = d["kc"], d["vc"]
            keys = g.view_3d(kc, hd, nkv, n_kv, g.h.ggml_row_size(F16, hd), kc.contents.nb[1], 0)
            kh = g.permute(keys, 0, 2, 1, 3)
            qh = g.permute(q, 0, 2, 1, 3)
            values = g.view_3d(vc, hd, nkv, n_kv, g.h.ggml_row_size(F16, hd), vc.contents.nb[1], 0)
            o = tap["att"] = g.flash_attn_ext(qh, kh, g.permute(values, 0, 2, 1, 3), self.mask, scale, 0.0, 0.0)
            g.h.ggml_flash_attn_ext_set_prec(o, 10)
            ao = tap["ao"] = g.mul_mat(d["wo"], g.reshape_2d(o, nq * hd, rows))
            x = tap["x1"] = g.add(x, ao)
            h = tap["h1"] = g.mul(g.rms_norm(x, eps), d["ffn_norm"])
            gate, up = g.mul_mat(d["w_gate"], h), g.mul_mat(d["w_up"], h)
            tap.update(gate=gate, up=up)
            g.expand(gate)
            g.expand(up)
            glu = tap["glu"] = g.swiglu_split(gate, up)
            dn = tap["dn"] = g.mul_mat(d["w_down"], glu)
            x = tap["x2"] = g.add(x, dn)
        self.hidden = g.mul(g.rms_norm(x, eps), self.out_norm)
        self.logits = g.mul_mat(self.head, self.hidden)
        self.pick = None
        if readback == "pick":
            self.pick = g.argmax(self.logits)
            g.h.ggml_set_output(self.pick)
            g.expand(self.pick)
        else:
            g.h.ggml_set_output(self.logits)
            g.h.ggml_set_output(self.hidden)
            g.expand(self.logits)
            g.expand(self.hidden)
        self.compute = g.tensors[n0:]

    def close(self):
        self.g.close()


def causal_mask(past, rows, n_kv):
    """Qwen3Decoder's mask (qwen3-decoder.cpp:64-70) as f16 bits [rows, n_kv]: row i sees positions 0 .. past + i."""
    m = np.where(np.arange(n_kv)[None, :] <= past + np.arange(rows)[:, None], 0.0, -np.inf).astype(np.float16)
    return m.view(np.uint16)
