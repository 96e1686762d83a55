"""Python binding of libmx (include/mx.h) through ctypes.

libmx is the product: C++ host code and hand-written gfx950 HIP kernels behind a C ABI. This module only binds that
ABI for the tests and the benchmark, the way a ctypes stub would bind it for any Python caller. It never computes
anything itself: if libmx.so is missing it raises, so nothing can pass on a fallback.

Tensors follow ggml order (ne[0] fastest). Device memory comes from the library's own buffers (mx_buffer_alloc).
"""
from __future__ import annotations

import ctypes
import os
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "libmx.so"

# ggml_type values
F32, F16, Q8_0, Q8_1, Q4_K, Q5_K, Q6_K, Q8_K, I32 = 0, 1, 8, 9, 12, 13, 14, 15, 26
BLCK = {F32: 1, F16: 1, I32: 1, Q8_0: 32, Q8_1: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256, Q8_K: 256}
TSIZE = {F32: 4, F16: 2, I32: 4, Q8_0: 34, Q8_1: 36, Q4_K: 144, Q5_K: 176, Q6_K: 210, Q8_K: 292}
# ggml types a model file may hold that the device keeps as plain bytes (Q4_0, Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, I8, I16,
# I64, F64, BF16)
BLCK.update({2: 32, 3: 32, 6: 32, 7: 32, 10: 256, 11: 256, 24: 1, 25: 1, 27: 1, 28: 1, 30: 1})
TSIZE.update({2: 18, 3: 20, 6: 22, 7: 24, 10: 84, 11: 110, 24: 1, 25: 2, 27: 8, 28: 8, 30: 2})
OP_GET_ROWS, OP_MUL_MAT, OP_MUL_MAT_ID, OP_ARGMAX = 1, 2, 3, 4
OP_RMS_NORM, OP_ADD, OP_MUL, OP_SWIGLU, OP_SET_ROWS = 5, 6, 7, 8, 9
ROPE_NEOX = 2
ROUND_REF, ROUND_X86 = 0, 1
# mx_backend_set_option keys (include/mx.h MX_OPT_*)
OPTIONS = {"gemm_q8_0": 1, "gemm_kquant": 2, "tile_m": 3, "tile_n": 4, "split": 5, "matvec_lpr": 6, "mmid_kernel": 7,
           "mmid_matvec_pairs": 8, "mmid_chunk": 9}
SUCCESS, FAILED, ALLOC_FAILED, INVALID, UNSUPPORTED = 0, -1, -2, -3, -4

EXPORTS = [
    "mx_device_count", "mx_device_description", "mx_device_memory", "mx_backend_init", "mx_backend_free",
    "mx_backend_stream", "mx_backend_synchronize", "mx_backend_set_rounding", "mx_backend_set_option",
    "mx_backend_get_option", "mx_last_error", "mx_buft_alignment",
    "mx_buft_max_size", "mx_tensor_alloc_size", "mx_buffer_alloc", "mx_buffer_free", "mx_buffer_clear",
    "mx_tensor_set", "mx_tensor_get", "mx_tensor_memset", "mx_tensor_copy", "mx_supports_op", "mx_get_rows",
    "mx_mul_mat", "mx_mul_mat_id", "mx_mul_mat_id_group", "mx_mul_mat_group", "mx_argmax", "mx_quantize_act", "mx_graph_begin", "mx_graph_end",
    "mx_graph_launch", "mx_graph_free", "mx_event_new", "mx_event_record", "mx_event_synchronize",
    "mx_event_elapsed_ms", "mx_event_free", "mx_quantize_chunk", "mx_fill_normal_rows", "mx_quantize_normal_rows",
    "mx_gguf_open", "mx_gguf_close", "mx_gguf_data_offset", "mx_gguf_n_tensors", "mx_gguf_get_tensor",
    "mx_gguf_find_tensor", "mx_gguf_n_keys", "mx_gguf_key", "mx_gguf_find_key", "mx_gguf_key_type", "mx_gguf_get_str",
    "mx_gguf_get_int", "mx_gguf_get_float", "mx_gguf_get_arr", "mx_gguf_get_arr_str", "mx_gguf_load_tensor",
    "mx_rms_norm", "mx_binary", "mx_swiglu", "mx_supports_rope", "mx_rope", "mx_set_rows", "mx_supports_flash_attn_ext",
    "mx_flash_attn_ext", "mx_mul_mat_fused", "mx_qk_norm_rope_kv", "mx_attn_decode", "mx_graph_nodes", "mx_mul_mat_id_noalloc", "mx_mul_mat_id_noalloc_bytes", "mx_peak_read", "mx_peak_mfma",
]
NOALLOC_SCRATCH_BYTES = 16 << 20  # MX_NOALLOC_SCRATCH_BYTES


def row_size(t: int, ne0: int) -> int:
    return ne0 // BLCK[t] * TSIZE[t]


class MxTensor(ctypes.Structure):
    _fields_ = [("type", ctypes.c_int32), ("pad_", ctypes.c_int32), ("ne", ctypes.c_int64 * 4),
                ("nb", ctypes.c_uint64 * 4), ("data", ctypes.c_void_p)]


class MxFusion(ctypes.Structure):
    _fields_ = [("norm_w", ctypes.POINTER(MxTensor)), ("norm_eps", ctypes.c_float),
                ("glu_b", ctypes.POINTER(MxTensor)), ("residual", ctypes.POINTER(ctypes.POINTER(MxTensor)))]


_P = ctypes.POINTER(MxTensor)


class GgufTensorInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("type", ctypes.c_int32), ("n_dims", ctypes.c_int32),
                ("ne", ctypes.c_int64 * 4), ("offset", ctypes.c_uint64), ("nbytes", ctypes.c_uint64)]


class MxError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"libmx status {code}: {msg}")
        self.code = code


def build(force: bool = True) -> None:
    """Compile libmx.so in-tree with hipcc for gfx950."""
    args = ["make", "-s", "-j8", "-C", str(HERE)]
    if force:
        args.insert(2, "-B")
    subprocess.run(args, check=True)


_lib = None


def lib():
    """The loaded libmx.so; raises if it has not been built (no fallback exists)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `make -C {HERE}` (or __graft_entry__.build())")
    L = ctypes.CDLL(str(LIB_PATH))
    vp, i32, i64, u64, sz, f32 = (ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_uint64, ctypes.c_size_t,
                                  ctypes.c_float)
    P = ctypes.POINTER(MxTensor)
    sig = {
        "mx_device_count": ([], i32),
        "mx_device_description": ([i32, ctypes.c_char_p, sz], i32),
        "mx_device_memory": ([i32, ctypes.POINTER(sz), ctypes.POINTER(sz)], i32),
        "mx_backend_init": ([i32], vp),
        "mx_backend_free": ([vp], None),
        "mx_backend_stream": ([vp], vp),
        "mx_backend_synchronize": ([vp], i32),
        "mx_backend_set_rounding": ([vp, i32], i32),
        "mx_backend_set_option": ([vp, i32, i64], i32),
        "mx_backend_get_option": ([vp, i32, ctypes.POINTER(i64)], i32),
        "mx_last_error": ([], ctypes.c_char_p),
        "mx_buft_alignment": ([], sz),
        "mx_buft_max_size": ([], sz),
        "mx_tensor_alloc_size": ([P], sz),
        "mx_buffer_alloc": ([vp, sz, ctypes.POINTER(vp)], i32),
        "mx_buffer_free": ([vp, vp], i32),
        "mx_buffer_clear": ([vp, vp, sz, ctypes.c_uint8], i32),
        "mx_tensor_set": ([vp, P, vp, sz, sz], i32),
        "mx_tensor_get": ([vp, P, vp, sz, sz], i32),
        "mx_tensor_memset": ([vp, P, ctypes.c_uint8, sz, sz], i32),
        "mx_tensor_copy": ([vp, P, P], i32),
        "mx_supports_op": ([i32, P, P, P, P], i32),
        "mx_get_rows": ([vp, P, P, P], i32),
        "mx_argmax": ([vp, P, P], i32),
        "mx_mul_mat": ([vp, P, P, P], i32),
        "mx_mul_mat_id": ([vp, P, P, P, P], i32),
        "mx_mul_mat_group": ([vp, i32, ctypes.POINTER(P), P, ctypes.POINTER(P)], i32),
        "mx_mul_mat_id_group": ([vp, i32, ctypes.POINTER(P), P, P, ctypes.POINTER(P)], i32),
        "mx_quantize_act": ([vp, i32, i32, vp, i64, i64, sz, vp], i32),
        "mx_peak_read": ([vp, vp, sz, i32, i32, i32], i32),
        "mx_peak_mfma": ([vp, i32, i32, i32], i32),
        "mx_graph_begin": ([vp], i32),
        "mx_graph_end": ([vp, ctypes.POINTER(vp)], i32),
        "mx_graph_launch": ([vp, vp], i32),
        "mx_graph_free": ([vp], None),
        "mx_event_new": ([vp], vp),
        "mx_event_record": ([vp, vp], i32),
        "mx_event_synchronize": ([vp], i32),
        "mx_event_elapsed_ms": ([vp, vp, ctypes.POINTER(f32)], i32),
        "mx_event_free": ([vp], None),
        "mx_quantize_chunk": ([i32, vp, vp, i64, i64, i64], sz),
        "mx_fill_normal_rows": ([u64, i64, i64, i64, f32, f32, vp], None),
        "mx_quantize_normal_rows": ([i32, u64, i64, i64, i64, f32, f32, vp, i32], sz),
        "mx_gguf_open": ([ctypes.c_char_p], vp),
        "mx_gguf_close": ([vp], None),
        "mx_gguf_data_offset": ([vp], u64),
        "mx_gguf_n_tensors": ([vp], i64),
        "mx_gguf_get_tensor": ([vp, i64, ctypes.POINTER(GgufTensorInfo)], i32),
        "mx_gguf_find_tensor": ([vp, ctypes.c_char_p], i64),
        "mx_gguf_n_keys": ([vp], i64),
        "mx_gguf_key": ([vp, i64], ctypes.c_char_p),
        "mx_gguf_find_key": ([vp, ctypes.c_char_p], i64),
        "mx_gguf_key_type": ([vp, i64], i32),
        "mx_gguf_get_str": ([vp, i64, ctypes.POINTER(vp), ctypes.POINTER(sz)], i32),
        "mx_gguf_get_int": ([vp, i64, ctypes.POINTER(i64)], i32),
        "mx_gguf_get_float": ([vp, i64, ctypes.POINTER(ctypes.c_double)], i32),
        "mx_gguf_get_arr": ([vp, i64, ctypes.POINTER(i32), ctypes.POINTER(u64), ctypes.POINTER(vp)], i32),
        "mx_gguf_get_arr_str": ([vp, i64, u64, ctypes.POINTER(vp), ctypes.POINTER(sz)], i32),
        "mx_gguf_load_tensor": ([vp, vp, i64, P], i32),
        "mx_rms_norm": ([vp, P, P, f32, P], i32),
        "mx_binary": ([vp, i32, P, P, P], i32),
        "mx_swiglu": ([vp, P, P, P], i32),
        "mx_supports_rope": ([P, P, P, i32, i32, f32, f32], i32),
        "mx_rope": ([vp, P, P, P, i32, i32, f32, f32, f32, f32], i32),
        "mx_set_rows": ([vp, P, P, P], i32),
        "mx_supports_flash_attn_ext": ([P, P, P, P, P, f32, f32], i32),
        "mx_flash_attn_ext": ([vp, P, P, P, P, P, f32], i32),
        "mx_mul_mat_fused": ([vp, i32, ctypes.POINTER(P), P, ctypes.POINTER(P), ctypes.POINTER(MxFusion)], i32),
        "mx_qk_norm_rope_kv": ([vp, P, P, P, P, P, P, P, P, P, f32, i32, i32, f32, f32, f32, f32], i32),
        "mx_attn_decode": ([vp, P, P, P, P, P, P, P, P, P, P, P, P, f32, i32, i32, f32, f32, f32, f32, f32], i32),
        "mx_graph_nodes": ([vp], sz),
        "mx_mul_mat_id_noalloc": ([vp, P, P, P, P], i32),
        "mx_mul_mat_id_noalloc_bytes": ([P, P, P], sz),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes, fn.restype = args, res
    _lib = L
    return L


def check(rc: int) -> None:
    if rc != SUCCESS:
        raise MxError(rc, lib().mx_last_error().decode(errors="replace"))


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ------------------------------------------------------------------------------------------ host-side quantization
def quantize_chunk(t: int, x: np.ndarray) -> np.ndarray:
    """ggml_quantize_chunk over a 2-D float32 matrix [nrows, n_per_row] (the library's host quantizer)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    nrows, npr = x.shape
    out = np.zeros((nrows, row_size(t, npr)), dtype=np.uint8)
    n = lib().mx_quantize_chunk(t, _p(x), _p(out), 0, nrows, npr)
    if n != out.size:
        raise ValueError("mx_quantize_chunk failed")
    return out


def fill_normal(seed: int, nrows: int, n_per_row: int, mean: float = 0.0, std: float = 1.0, row0: int = 0):
    out = np.empty((nrows, n_per_row), dtype=np.float32)
    lib().mx_fill_normal_rows(seed & (2**64 - 1), row0, nrows, n_per_row, mean, std, _p(out))
    return out


def quantize_normal(t: int, seed: int, nrows: int, n_per_row: int, std: float, nthreads: int | None = None,
                    mean: float = 0.0, row0: int = 0) -> np.ndarray:
    out = np.empty((nrows, row_size(t, n_per_row)), dtype=np.uint8)
    nthreads = nthreads or max(1, len(os.sched_getaffinity(0)))
    n = lib().mx_quantize_normal_rows(t, seed & (2**64 - 1), row0, nrows, n_per_row, mean, std, _p(out), nthreads)
    if n != out.size:
        raise ValueError("mx_quantize_normal_rows failed")
    return out


# ------------------------------------------------------------------------------------------------------ device side
def contiguous_nb(t: int, ne) -> tuple:
    nb0 = TSIZE[t]
    nb1 = row_size(t, ne[0])
    nb2 = nb1 * ne[1]
    nb3 = nb2 * ne[2]
    return (nb0, nb1, nb2, nb3)


class Tensor:
    """A ggml-shaped tensor in a buffer of its own on the device."""

    def __init__(self, be: "Backend", t: int, ne, nb=None):
        ne = tuple(int(v) for v in ne) + (1,) * (4 - len(ne))
        self.be = be
        self.type = t
        self.ne = ne
        self.desc = MxTensor()
        self.desc.type = t
        for i in range(4):
            self.desc.ne[i] = ne[i]
        nb = nb or contiguous_nb(t, ne)
        for i in range(4):
            self.desc.nb[i] = nb[i]
        self.size = int(lib().mx_tensor_alloc_size(ctypes.byref(self.desc)))
        base = ctypes.c_void_p()
        check(lib().mx_buffer_alloc(be.h, max(self.size, 256), ctypes.byref(base)))
        self.base = base.value
        self.desc.data = self.base
        self.nbytes = row_size(t, ne[0]) * ne[1] * ne[2] * ne[3]

    def ref(self):
        return ctypes.byref(self.desc)

    def view(self, ne, nb, offset: int = 0) -> "View":
        """A ggml view of this tensor's memory (ggml_view_* / ggml_permute): other ne / nb, same bytes."""
        return View(self, ne, nb, offset)

    def set(self, data: np.ndarray, offset: int = 0) -> "Tensor":
        data = np.ascontiguousarray(data)
        check(lib().mx_tensor_set(self.be.h, self.ref(), _p(data), offset, data.nbytes))
        return self

    def get_bytes(self, offset: int = 0, size: int | None = None) -> np.ndarray:
        size = self.nbytes - offset if size is None else size
        out = np.empty(size, dtype=np.uint8)
        check(lib().mx_tensor_get(self.be.h, self.ref(), _p(out), offset, size))
        return out

    def numpy(self) -> np.ndarray:
        """Contents in ggml order, shaped [ne3, ne2, ne1, ne0] (f32 / i32) or [.., row bytes] (quantized)."""
        b = self.get_bytes()
        shape = (self.ne[3], self.ne[2], self.ne[1])
        if self.type == F32:
            return b.view(np.float32).reshape(shape + (self.ne[0],))
        if self.type == I32:
            return b.view(np.int32).reshape(shape + (self.ne[0],))
        return b.reshape(shape + (row_size(self.type, self.ne[0]),))

    def free(self) -> None:
        if self.base:
            check(lib().mx_buffer_free(self.be.h, self.base))
            self.base = None

    def __del__(self):
        try:
            if self.base and self.be.h:
                lib().mx_buffer_free(self.be.h, self.base)
        except Exception:
            pass


class View:
    """A tensor descriptor over another tensor's memory (owns nothing)."""

    def __init__(self, base: Tensor, ne, nb, offset: int = 0):
        ne = tuple(int(v) for v in ne) + (1,) * (4 - len(ne))
        nb = tuple(int(v) for v in nb) + (nb[-1] * ne[len(nb) - 1],) * (4 - len(nb))
        self.base_tensor = base
        self.type = base.type
        self.ne = ne
        self.desc = MxTensor()
        self.desc.type = base.type
        for i in range(4):
            self.desc.ne[i] = ne[i]
            self.desc.nb[i] = nb[i]
        self.desc.data = base.base + offset

    def ref(self):
        return ctypes.byref(self.desc)


class Backend:
    """One device backend: a HIP stream, scratch and an error word (ggml_backend_t)."""

    def __init__(self, device: int = 0):
        L = lib()
        self.h = L.mx_backend_init(device)
        if not self.h:
            raise MxError(FAILED, L.mx_last_error().decode())
        self.device = device

    def close(self) -> None:
        if self.h:
            lib().mx_backend_free(self.h)
            self.h = None

    def tensor(self, t: int, ne, data: np.ndarray | None = None) -> Tensor:
        T = Tensor(self, t, ne)
        if data is not None:
            T.set(data)
        return T

    def sync(self) -> None:
        check(lib().mx_backend_synchronize(self.h))

    def set_rounding(self, r: int) -> None:
        check(lib().mx_backend_set_rounding(self.h, r))

    def set_option(self, name: str, value: int) -> None:
        """A kernel choice of this backend (mx_backend_set_option; names are the keys of OPTIONS)."""
        check(lib().mx_backend_set_option(self.h, OPTIONS[name], int(value)))

    def get_option(self, name: str) -> int:
        v = ctypes.c_int64()
        check(lib().mx_backend_get_option(self.h, OPTIONS[name], ctypes.byref(v)))
        return int(v.value)

    def options(self, **kw):
        """Context manager: the given options set for the block, the previous values restored after it."""
        import contextlib

        @contextlib.contextmanager
        def cm():
            old = {k: self.get_option(k) for k in kw}
            try:
                for k, v in kw.items():
                    self.set_option(k, v)
                yield self
            finally:
                for k, v in old.items():
                    self.set_option(k, v)
        return cm()

    def get_rows(self, src0: Tensor, ids: Tensor, dst: Tensor) -> None:
        check(lib().mx_get_rows(self.h, src0.ref(), ids.ref(), dst.ref()))

    def mul_mat(self, src0: Tensor, src1: Tensor, dst: Tensor) -> None:
        check(lib().mx_mul_mat(self.h, src0.ref(), src1.ref(), dst.ref()))

    def mul_mat_group(self, src0s, src1: Tensor, dsts) -> None:
        P = ctypes.POINTER(MxTensor)
        a = (P * len(src0s))(*[ctypes.pointer(s.desc) for s in src0s])
        d = (P * len(dsts))(*[ctypes.pointer(s.desc) for s in dsts])
        check(lib().mx_mul_mat_group(self.h, len(src0s), a, src1.ref(), d))

    def mul_mat_id(self, as_: Tensor, b: Tensor, ids: Tensor, dst: Tensor) -> None:
        check(lib().mx_mul_mat_id(self.h, as_.ref(), b.ref(), ids.ref(), dst.ref()))

    def mul_mat_id_group(self, as_list, b: Tensor, ids: Tensor, dsts) -> None:
        """n MUL_MAT_IDs sharing b and ids (gate and up experts) with one prep launch."""
        P = ctypes.POINTER(MxTensor)
        w = (P * len(as_list))(*[ctypes.pointer(t.desc) for t in as_list])
        y = (P * len(dsts))(*[ctypes.pointer(d.desc) for d in dsts])
        check(lib().mx_mul_mat_id_group(self.h, len(as_list), w, b.ref(), ids.ref(), y))

    def mul_mat_id_noalloc(self, as_: Tensor, b: Tensor, ids: Tensor, dst: Tensor) -> None:
        """MUL_MAT_ID on the GPU's static scratch: allocates nothing (mx_mul_mat_id_noalloc)."""
        check(lib().mx_mul_mat_id_noalloc(self.h, as_.ref(), b.ref(), ids.ref(), dst.ref()))

    def argmax(self, src: Tensor, dst: Tensor) -> None:
        check(lib().mx_argmax(self.h, src.ref(), dst.ref()))

    def mul_mat_fused(self, src0s, src1, dsts, norm_w=None, eps: float = 0.0, glu_b=None, residual=None) -> None:
        """dst[i] = residual[i] + src0[i] x f(src1), f = mul(rms_norm(., eps), norm_w) and / or swiglu(., glu_b)."""
        P = ctypes.POINTER(MxTensor)
        w = (P * len(src0s))(*[ctypes.pointer(s.desc) for s in src0s])
        y = (P * len(dsts))(*[ctypes.pointer(d.desc) for d in dsts])
        f = MxFusion()
        f.norm_w = ctypes.pointer(norm_w.desc) if norm_w is not None else None
        f.norm_eps = eps
        f.glu_b = ctypes.pointer(glu_b.desc) if glu_b is not None else None
        res = None
        if residual is not None:
            res = (P * len(residual))(*[ctypes.pointer(r.desc) if r is not None else None for r in residual])
            f.residual = ctypes.cast(res, ctypes.POINTER(P))
        check(lib().mx_mul_mat_fused(self.h, len(src0s), w, src1.ref(), y, ctypes.byref(f)))

    def qk_norm_rope_kv(self, q, k, v, q_norm, k_norm, pos, q_out, k_cache, v_cache, eps: float, freq_base: float,
                        n_dims: int = 128, freq_scale: float = 1.0) -> None:
        check(lib().mx_qk_norm_rope_kv(self.h, q.ref(), k.ref(), v.ref(), q_norm.ref(), k_norm.ref(), pos.ref(),
                                       q_out.ref(), k_cache.ref(), v_cache.ref(), eps, n_dims, ROPE_NEOX, freq_base,
                                       freq_scale, 0.0, 1.0))

    def attn_decode(self, q, k, v, q_norm, k_norm, pos, k_cache, v_cache, k_view, v_view, mask, dst, eps: float,
                    freq_base: float, scale: float, n_dims: int = 128, freq_scale: float = 1.0) -> None:
        """qk_norm_rope_kv then flash_attn_ext over the caches, for one decode row, in one launch."""
        check(lib().mx_attn_decode(self.h, q.ref(), k.ref(), v.ref(), q_norm.ref(), k_norm.ref(), pos.ref(),
                                   k_cache.ref(), v_cache.ref(), k_view.ref(), v_view.ref(),
                                   mask.ref() if mask is not None else None, dst.ref(), eps, n_dims, ROPE_NEOX,
                                   freq_base, freq_scale, 0.0, 1.0, scale))

    def rms_norm(self, src: Tensor, dst: Tensor, eps: float, w: Tensor | None = None) -> None:
        check(lib().mx_rms_norm(self.h, src.ref(), dst.ref(), eps, w.ref() if w is not None else None))

    def add(self, a: Tensor, b: Tensor, dst: Tensor) -> None:
        check(lib().mx_binary(self.h, OP_ADD, a.ref(), b.ref(), dst.ref()))

    def mul(self, a: Tensor, b: Tensor, dst: Tensor) -> None:
        check(lib().mx_binary(self.h, OP_MUL, a.ref(), b.ref(), dst.ref()))

    def swiglu(self, a: Tensor, b: Tensor, dst: Tensor) -> None:
        check(lib().mx_swiglu(self.h, a.ref(), b.ref(), dst.ref()))

    def rope(self, src: Tensor, pos: Tensor, dst: Tensor, n_dims: int, freq_base: float, freq_scale: float = 1.0,
             mode: int = ROPE_NEOX) -> None:
        check(lib().mx_rope(self.h, src.ref(), pos.ref(), dst.ref(), n_dims, mode, freq_base, freq_scale, 0.0, 1.0))

    def set_rows(self, src: Tensor, idx: Tensor, dst: Tensor) -> None:
        check(lib().mx_set_rows(self.h, src.ref(), idx.ref(), dst.ref()))

    def flash_attn_ext(self, q: Tensor, k: Tensor, v: Tensor, mask: Tensor | None, dst: Tensor, scale: float) -> None:
        check(lib().mx_flash_attn_ext(self.h, q.ref(), k.ref(), v.ref(), mask.ref() if mask is not None else None,
                                      dst.ref(), scale))

    def quantize_act(self, t: int, rounding: int, x: Tensor, k: int, nrows: int) -> Tensor:
        out = Tensor(self, F32, (row_size(t, k) * nrows // 4 + 1,))
        check(lib().mx_quantize_act(self.h, t, rounding, ctypes.c_void_p(x.base), k, nrows, x.desc.nb[1],
                                    ctypes.c_void_p(out.base)))
        return out

    def peak_read(self, src: Tensor, workgroups: int, loads: int, nontemporal: bool = False) -> None:
        """One streaming read of all of src's bytes (mx_peak_read)."""
        check(lib().mx_peak_read(self.h, ctypes.c_void_p(src.base), src.nbytes, workgroups, loads, int(nontemporal)))

    def peak_mfma(self, kind: int, workgroups: int, iters: int) -> None:
        """Rounds of independent MFMAs on register operands (mx_peak_mfma): kind 0 int8, 1 fp16."""
        check(lib().mx_peak_mfma(self.h, kind, workgroups, iters))

    def supports(self, op: int, src0: Tensor, src1: Tensor | None, src2: Tensor | None, dst: Tensor) -> bool:
        r = lambda t: t.ref() if t is not None else None  # noqa: E731
        return bool(lib().mx_supports_op(op, r(src0), r(src1), r(src2), r(dst)))

    # graphs and events
    def graph_begin(self) -> None:
        check(lib().mx_graph_begin(self.h))

    def graph_end(self):
        g = ctypes.c_void_p()
        check(lib().mx_graph_end(self.h, ctypes.byref(g)))
        return g.value

    def graph_launch(self, g) -> None:
        check(lib().mx_graph_launch(self.h, ctypes.c_void_p(g)))

    @staticmethod
    def graph_nodes(g) -> int:
        return int(lib().mx_graph_nodes(ctypes.c_void_p(g)))

    def graph_free(self, g) -> None:
        lib().mx_graph_free(ctypes.c_void_p(g))

    def event(self):
        e = lib().mx_event_new(self.h)
        if not e:
            raise MxError(FAILED, lib().mx_last_error().decode())
        return e

    def record(self, e) -> None:
        check(lib().mx_event_record(self.h, ctypes.c_void_p(e)))

    @staticmethod
    def elapsed_ms(e0, e1) -> float:
        check(lib().mx_event_synchronize(ctypes.c_void_p(e1)))
        ms = ctypes.c_float()
        check(lib().mx_event_elapsed_ms(ctypes.c_void_p(e0), ctypes.c_void_p(e1), ctypes.byref(ms)))
        return float(ms.value)

    @staticmethod
    def event_free(e) -> None:
        lib().mx_event_free(ctypes.c_void_p(e))


def device_count() -> int:
    return int(lib().mx_device_count())


def device_description(device: int = 0) -> str:
    buf = ctypes.create_string_buffer(256)
    check(lib().mx_device_description(device, buf, 256))
    return buf.value.decode()


# ------------------------------------------------------------------------------------------------------------ GGUF
GGUF_ARRAY_DTYPES = {0: np.uint8, 1: np.int8, 2: np.uint16, 3: np.int16, 4: np.uint32, 5: np.int32, 6: np.float32,
                     7: np.bool_, 10: np.uint64, 11: np.int64, 12: np.float64}


class Gguf:
    """A GGUF file parsed by libmx (mx_gguf_open): metadata, tensor infos, and tensors read into a backend's buffer
    type in 16 MB pieces (mx_gguf_load_tensor) -- what speech.cpp's ModelFile::open / load do through ggml."""

    def __init__(self, path):
        self.h = lib().mx_gguf_open(str(path).encode())
        if not self.h:
            raise MxError(FAILED, lib().mx_last_error().decode(errors="replace"))

    def close(self) -> None:
        if self.h:
            lib().mx_gguf_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def data_offset(self) -> int:
        return int(lib().mx_gguf_data_offset(self.h))

    def tensors(self) -> list:
        out = []
        for i in range(lib().mx_gguf_n_tensors(self.h)):
            info = GgufTensorInfo()
            check(lib().mx_gguf_get_tensor(self.h, i, ctypes.byref(info)))
            out.append({"name": info.name.decode(), "type": info.type, "n_dims": info.n_dims, "ne": tuple(info.ne),
                        "offset": int(info.offset), "nbytes": int(info.nbytes)})
        return out

    def find_tensor(self, name: str) -> int:
        return int(lib().mx_gguf_find_tensor(self.h, name.encode()))

    def keys(self) -> list:
        return [lib().mx_gguf_key(self.h, i).decode() for i in range(lib().mx_gguf_n_keys(self.h))]

    def get(self, key: str):
        """The value of a key (None if absent): int, float, str, or a list / numpy array for arrays."""
        L = lib()
        i = L.mx_gguf_find_key(self.h, key.encode())
        if i < 0:
            return None
        vt = L.mx_gguf_key_type(self.h, i)
        if vt == 8:
            p, n = ctypes.c_void_p(), ctypes.c_size_t()
            check(L.mx_gguf_get_str(self.h, i, ctypes.byref(p), ctypes.byref(n)))
            return ctypes.string_at(p.value, n.value).decode() if n.value else ""
        if vt in (6, 12):
            v = ctypes.c_double()
            check(L.mx_gguf_get_float(self.h, i, ctypes.byref(v)))
            return v.value
        if vt == 9:
            et, n, data = ctypes.c_int(), ctypes.c_uint64(), ctypes.c_void_p()
            check(L.mx_gguf_get_arr(self.h, i, ctypes.byref(et), ctypes.byref(n), ctypes.byref(data)))
            if et.value == 8:
                out = []
                for j in range(n.value):
                    p, m = ctypes.c_void_p(), ctypes.c_size_t()
                    check(L.mx_gguf_get_arr_str(self.h, i, j, ctypes.byref(p), ctypes.byref(m)))
                    out.append(ctypes.string_at(p.value, m.value).decode() if m.value else "")
                return out
            dt = np.dtype(GGUF_ARRAY_DTYPES[et.value])
            if n.value == 0:
                return np.zeros(0, dt)
            return np.frombuffer(ctypes.string_at(data.value, n.value * dt.itemsize), dt).copy()
        v = ctypes.c_int64()
        check(L.mx_gguf_get_int(self.h, i, ctypes.byref(v)))
        return bool(v.value) if vt == 7 else v.value

    def load(self, be: "Backend", name: str) -> "Tensor":
        """Allocates the named tensor in the backend's buffer type and reads it from the file."""
        i = self.find_tensor(name)
        if i < 0:
            raise KeyError(name)
        info = self.tensors()[i]
        T = be.tensor(info["type"], info["ne"])
        check(lib().mx_gguf_load_tensor(be.h, self.h, i, T.ref()))
        return T
