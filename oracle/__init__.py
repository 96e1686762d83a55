"""ctypes wrapper of the CPU oracle (mx_oracle.c) and of the AVX2 CPU-baseline port (cpu_fast.c).

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this package, and
only as the checker or the timed CPU baseline; the product (libmx) never calls it.

All byte buffers are numpy uint8 arrays in ggml's block layout; tensors follow ggml order (ne[0] fastest).
"""
from __future__ import annotations

import ctypes
import os
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
BUILD = HERE / "_build"

TYPE_F32, TYPE_F16, TYPE_Q8_0, TYPE_Q8_1, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_K, TYPE_I32 = \
    0, 1, 8, 9, 12, 13, 14, 15, 26
ROUND_REF, ROUND_X86 = 0, 1

BLCK = {TYPE_F32: 1, TYPE_F16: 1, TYPE_I32: 1, TYPE_Q8_0: 32, TYPE_Q8_1: 32, TYPE_Q4_K: 256, TYPE_Q5_K: 256,
        TYPE_Q6_K: 256, TYPE_Q8_K: 256}
TSIZE = {TYPE_F32: 4, TYPE_F16: 2, TYPE_I32: 4, TYPE_Q8_0: 34, TYPE_Q8_1: 36, TYPE_Q4_K: 144, TYPE_Q5_K: 176,
         TYPE_Q6_K: 210, TYPE_Q8_K: 292}
VEC_DOT_TYPE = {TYPE_Q8_0: TYPE_Q8_0, TYPE_Q4_K: TYPE_Q8_K, TYPE_Q5_K: TYPE_Q8_K, TYPE_Q6_K: TYPE_Q8_K,
                TYPE_F16: TYPE_F16, TYPE_F32: TYPE_F32}


def row_size(t: int, ne0: int) -> int:
    return ne0 // BLCK[t] * TSIZE[t]


class OrcTensor(ctypes.Structure):
    _fields_ = [("type", ctypes.c_int32), ("ne", ctypes.c_int64 * 4), ("nb", ctypes.c_size_t * 4),
                ("data", ctypes.c_void_p)]


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


_lib = None
_fast = None


def lib():
    global _lib
    if _lib is None:
        path = BUILD / "liboracle.so"
        if not path.exists():
            build()
        L = ctypes.CDLL(str(path))
        vp, i64, u64, f32, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_uint64, ctypes.c_float, ctypes.c_int
        L.orc_fp32_to_fp16.argtypes, L.orc_fp32_to_fp16.restype = [f32], ctypes.c_uint16
        L.orc_fp16_to_fp32.argtypes, L.orc_fp16_to_fp32.restype = [ctypes.c_uint16], f32
        for n in ("orc_quantize_row_q8_0", "orc_quantize_row_q8_1"):
            getattr(L, n).argtypes, getattr(L, n).restype = [vp, vp, i64, i32], None
        for n in ("orc_quantize_row_q8_K", "orc_quantize_row_q4_K", "orc_quantize_row_q5_K", "orc_quantize_row_q6_K"):
            getattr(L, n).argtypes, getattr(L, n).restype = [vp, vp, i64], None
        L.orc_quantize_chunk.argtypes, L.orc_quantize_chunk.restype = [i32, vp, vp, i64, i64, i64], ctypes.c_size_t
        L.orc_make_qkx2_quants.argtypes = [i32, i32, vp, vp, vp, vp, f32, f32, i32, i32]
        L.orc_make_qkx2_quants.restype = f32
        L.orc_make_qx_quants.argtypes, L.orc_make_qx_quants.restype = [i32, i32, vp, vp], f32
        L.orc_dequantize_row.argtypes, L.orc_dequantize_row.restype = [i32, vp, vp, i64], i32
        L.orc_vec_dot.argtypes, L.orc_vec_dot.restype = [i32, i64, vp, vp], f32
        L.orc_vec_dot_exact.argtypes, L.orc_vec_dot_exact.restype = [i32, i64, vp, vp], ctypes.c_double
        P = ctypes.POINTER(OrcTensor)
        L.orc_mul_mat.argtypes, L.orc_mul_mat.restype = [P, P, P, i32, i32], i32
        L.orc_mul_mat_id.argtypes, L.orc_mul_mat_id.restype = [P, P, P, P, i32, i32], i32
        L.orc_get_rows.argtypes, L.orc_get_rows.restype = [P, P, P], i32
        L.orc_argmax.argtypes, L.orc_argmax.restype = [P, P], i32
        L.orc_rms_norm.argtypes, L.orc_rms_norm.restype = [vp, vp, i64, i64, f32], None
        L.orc_binary.argtypes, L.orc_binary.restype = [i32, vp, vp, vp, i64, i64, i64], None
        L.orc_swiglu.argtypes, L.orc_swiglu.restype = [vp, vp, vp, i64], None
        L.orc_rope_neox.argtypes, L.orc_rope_neox.restype = [vp, vp, vp, i64, i64, i64, i32, f32, f32], None
        L.orc_set_rows_f16.argtypes, L.orc_set_rows_f16.restype = [vp, vp, vp, i64, i64, i64], i32
        L.orc_flash_attn_ext.argtypes = [vp, vp, vp, vp, vp, i32, i64, i64, i64, i64, f32, i32]
        L.orc_flash_attn_ext.restype = i32
        L.orc_fill_normal_rows.argtypes = [u64, i64, i64, i64, f32, f32, vp]
        L.orc_fill_normal_rows.restype = None
        _lib = L
    return _lib


def fast():
    global _fast
    if _fast is None:
        path = BUILD / "libcpufast.so"
        if not path.exists():
            build()
        F = ctypes.CDLL(str(path))
        P = ctypes.POINTER(OrcTensor)
        F.cpf_mul_mat.argtypes, F.cpf_mul_mat.restype = [P, P, P, ctypes.c_int], ctypes.c_int
        F.cpf_have_avx2.argtypes, F.cpf_have_avx2.restype = [], ctypes.c_int
        F.cpf_q8_0_isa.argtypes, F.cpf_q8_0_isa.restype = [], ctypes.c_int
        vp, i64 = ctypes.c_void_p, ctypes.c_int64
        F.cpf_flash_attn_ext.argtypes = [vp, vp, vp, vp, vp, ctypes.c_int, i64, i64, i64, i64, ctypes.c_float,
                                         ctypes.c_int]
        F.cpf_flash_attn_ext.restype = ctypes.c_int
        _fast = F
    return _fast


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ---------------------------------------------------------------------------------------------------------------- fp16
def fp32_to_fp16_bits(x: float) -> int:
    return int(lib().orc_fp32_to_fp16(float(x)))


def fp16_bits_to_fp32(h: int) -> float:
    return float(lib().orc_fp16_to_fp32(int(h)))


# ------------------------------------------------------------------------------------------------------- quantization
def quantize_rows(t: int, x: np.ndarray, rounding: int = ROUND_REF) -> np.ndarray:
    """Quantize each row of x (float32, [..., K]) to ggml type t; returns uint8 [..., row_size]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    K = x.shape[-1]
    rows = x.reshape(-1, K)
    out = np.zeros((rows.shape[0], row_size(t, K)), dtype=np.uint8)
    L = lib()
    for r in range(rows.shape[0]):
        src = rows[r]
        dst = out[r]
        if t == TYPE_Q8_0:
            L.orc_quantize_row_q8_0(_p(src), _p(dst), K, rounding)
        elif t == TYPE_Q8_1:
            L.orc_quantize_row_q8_1(_p(src), _p(dst), K, rounding)
        elif t == TYPE_Q8_K:
            L.orc_quantize_row_q8_K(_p(src), _p(dst), K)
        elif t == TYPE_Q4_K:
            L.orc_quantize_row_q4_K(_p(src), _p(dst), K)
        elif t == TYPE_Q5_K:
            L.orc_quantize_row_q5_K(_p(src), _p(dst), K)
        elif t in (TYPE_F16, TYPE_F32):
            L.orc_quantize_chunk(t, _p(src), _p(dst), 0, 1, K)
        elif t == TYPE_Q6_K:
            L.orc_quantize_row_q6_K(_p(src), _p(dst), K)
        else:
            raise ValueError(t)
    return out.reshape(x.shape[:-1] + (row_size(t, K),))


def quantize_chunk(t: int, x: np.ndarray) -> np.ndarray:
    """ggml_quantize_chunk over all rows of a 2-D float32 matrix [nrows, n_per_row] (imatrix = NULL)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    nrows, npr = x.shape
    out = np.zeros((nrows, row_size(t, npr)), dtype=np.uint8)
    n = lib().orc_quantize_chunk(t, _p(x), _p(out), 0, nrows, npr)
    if n != out.size:
        raise ValueError("quantize_chunk failed")
    return out


def make_qkx2_quants(x: np.ndarray, weights: np.ndarray, nmax: int, rmin: float, rdelta: float, nstep: int):
    """ggml's make_qkx2_quants on one sub-block (use_mad = 0): (scale, min, codes) with x ~ scale * code + min."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(weights, dtype=np.float32)
    L = np.zeros(x.size, np.uint8)
    neg_min = np.zeros(1, np.float32)
    scale = lib().orc_make_qkx2_quants(x.size, nmax, _p(x), _p(w), _p(L), _p(neg_min), rmin, rdelta, nstep, 0)
    return np.float32(scale), -neg_min[0], L


def make_qx_quants(x: np.ndarray, nmax: int):
    """ggml's make_qx_quants (rmse_type 1, no importance weights) on one sub-block: (scale, codes - nmax)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    L = np.zeros(x.size, np.int8)
    scale = lib().orc_make_qx_quants(x.size, nmax, _p(x), _p(L))
    return np.float32(scale), L.astype(np.int64) - nmax


def dequantize_rows(t: int, q: np.ndarray, K: int) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    rows = q.reshape(-1, row_size(t, K))
    out = np.zeros((rows.shape[0], K), dtype=np.float32)
    for r in range(rows.shape[0]):
        if lib().orc_dequantize_row(t, _p(rows[r]), _p(out[r]), K) != 0:
            raise ValueError(t)
    return out.reshape(q.shape[:-1] + (K,))


def vec_dot(t: int, K: int, wrow: np.ndarray, arow: np.ndarray, exact: bool = False) -> float:
    if exact:
        return float(lib().orc_vec_dot_exact(t, K, _p(wrow), _p(arow)))
    return float(lib().orc_vec_dot(t, K, _p(wrow), _p(arow)))


# ------------------------------------------------------------------------------------------------------------ tensors
def _tensor(t: int, arr: np.ndarray, ne: tuple) -> OrcTensor:
    ne = tuple(ne) + (1,) * (4 - len(ne))
    T = OrcTensor()
    T.type = t
    for i in range(4):
        T.ne[i] = ne[i]
    nb0 = TSIZE[t]
    T.nb[0] = nb0
    T.nb[1] = row_size(t, ne[0])
    T.nb[2] = T.nb[1] * ne[1]
    T.nb[3] = T.nb[2] * ne[2]
    T.data = _p(arr)
    return T


def mul_mat(wtype: int, w: np.ndarray, x: np.ndarray, rounding: int = ROUND_REF, exact: bool = False) -> np.ndarray:
    """ggml_mul_mat(W, X): w uint8 [(E,) N, row_size] quantized rows; x float32 [M, K] -> y float32 [M, N]."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    N = w.shape[0]
    y = np.zeros((M, N), dtype=np.float32)
    s0, s1, d = _tensor(wtype, w, (K, N)), _tensor(TYPE_F32, x, (K, M)), _tensor(TYPE_F32, y, (N, M))
    rc = lib().orc_mul_mat(ctypes.byref(s0), ctypes.byref(s1), ctypes.byref(d), rounding, int(exact))
    if rc != 0:
        raise ValueError(f"orc_mul_mat rc={rc}")
    return y


def mul_mat_par(wtype: int, w: np.ndarray, x: np.ndarray, rounding: int = ROUND_REF, threads: int = 0) -> np.ndarray:
    """mul_mat over row ranges of w on several host threads (ctypes releases the GIL during each call): the same
    oracle, the same per-output arithmetic, for products too large for one thread in a test's time."""
    from concurrent.futures import ThreadPoolExecutor

    threads = threads or physical_cores()
    N = w.shape[0]
    if threads <= 1 or N < 2 * threads:
        return mul_mat(wtype, w, x, rounding)
    step = (N + threads - 1) // threads
    parts = [(a, min(N, a + step)) for a in range(0, N, step)]
    with ThreadPoolExecutor(len(parts)) as ex:
        outs = list(ex.map(lambda r: mul_mat(wtype, np.ascontiguousarray(w[r[0]:r[1]]), x, rounding), parts))
    return np.concatenate(outs, axis=-1)


def mul_mat_id(wtype: int, w: np.ndarray, x: np.ndarray, ids: np.ndarray, rounding: int = ROUND_REF,
               exact: bool = False) -> np.ndarray:
    """ggml_mul_mat_id: w uint8 [E, N, row_size]; x float32 [T, B, K] (B = 1 or n_ids); ids int32 [T, n_ids]
    -> y float32 [T, n_ids, N]."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    E, N, _ = w.shape
    T, B, K = x.shape
    n_ids = ids.shape[1]
    y = np.zeros((T, n_ids, N), dtype=np.float32)
    s0 = _tensor(wtype, w, (K, N, E))
    s1 = _tensor(TYPE_F32, x, (K, B, T))
    si = _tensor(TYPE_I32, ids, (n_ids, T))
    d = _tensor(TYPE_F32, y, (N, n_ids, T))
    rc = lib().orc_mul_mat_id(ctypes.byref(s0), ctypes.byref(s1), ctypes.byref(si), ctypes.byref(d), rounding,
                              int(exact))
    if rc != 0:
        raise ValueError(f"orc_mul_mat_id rc={rc}")
    return y


def get_rows(wtype: int, table: np.ndarray, K: int, ids: np.ndarray) -> np.ndarray:
    """ggml_get_rows on a 2-D table: table uint8 [R, row_size]; ids int32 [n] -> float32 [n, K]."""
    table = np.ascontiguousarray(table, dtype=np.uint8)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    R = table.shape[0]
    out = np.zeros((ids.shape[0], K), dtype=np.float32)
    s0, si, d = _tensor(wtype, table, (K, R)), _tensor(TYPE_I32, ids, (ids.shape[0],)), _tensor(TYPE_F32, out, (K, ids.shape[0]))
    rc = lib().orc_get_rows(ctypes.byref(s0), ctypes.byref(si), ctypes.byref(d))
    if rc != 0:
        raise ValueError(f"orc_get_rows rc={rc}")
    return out


def argmax(x: np.ndarray) -> np.ndarray:
    """ggml_argmax with the first of equal values: x float32 [R, n] -> int32 [R]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.shape[0], dtype=np.int32)
    s0, d = _tensor(TYPE_F32, x, (x.shape[1], x.shape[0])), _tensor(TYPE_I32, out, (x.shape[0],))
    rc = lib().orc_argmax(ctypes.byref(s0), ctypes.byref(d))
    if rc != 0:
        raise ValueError(f"orc_argmax rc={rc}")
    return out


# ------------------------------------------------------------------------------------ the decoder layer's other ops
def rms_norm(x: np.ndarray, eps: float) -> np.ndarray:
    """ggml_rms_norm over the last axis of x (float32)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().orc_rms_norm(_p(x), _p(y), x.shape[-1], x.size // x.shape[-1], eps)
    return y


def binary(op: str, a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """ggml_add / ggml_mul (op "add" / "mul") with b's rows repeated over a's rows (last axis = ne0)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    ne0 = a.shape[-1]
    y = np.empty_like(a)
    lib().orc_binary(0 if op == "add" else 1, _p(a), _p(b), _p(y), ne0, a.size // ne0, b.size // ne0)
    return y


def swiglu(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    y = np.empty_like(a)
    lib().orc_swiglu(_p(a), _p(b), _p(y), a.size)
    return y


def rope_neox(x: np.ndarray, pos: np.ndarray, n_dims: int, freq_base: float, freq_scale: float = 1.0) -> np.ndarray:
    """ggml_rope_ext(NEOX) on x float32 [rows, n_head, ne0] with pos int32 [rows]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    rows, n_head, ne0 = x.shape
    y = np.empty_like(x)
    lib().orc_rope_neox(_p(x), _p(pos), _p(y), ne0, n_head, rows, n_dims, freq_base, freq_scale)
    return y


def set_rows_f16(cache: np.ndarray, src: np.ndarray, idx: np.ndarray) -> np.ndarray:
    """ggml_set_rows into an f16 cache: cache uint16 [R, ne0] (copied), src float32 [n, ne0], idx int32 [n]."""
    out = np.ascontiguousarray(cache, dtype=np.uint16).copy()
    src = np.ascontiguousarray(src, dtype=np.float32)
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    if lib().orc_set_rows_f16(_p(src), _p(idx), _p(out), src.shape[1], src.shape[0], out.shape[0]) != 0:
        raise ValueError("set_rows index out of range")
    return out


def flash_attn_ext(q: np.ndarray, k: np.ndarray, v: np.ndarray, mask, scale: float, exact: bool = False):
    """ggml_flash_attn_ext: q float32 [n_head, n_q, D]; k, v uint16 (fp16 bits) [n_kv_head, n_kv, D]; mask uint16
    [n_q, n_kv] or None -> float32 [n_q, n_head, D] (the permuted output the decoder reshapes)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    n_head, n_q, D = q.shape
    n_kv_head, n_kv, _ = k.shape
    out = np.zeros((n_q, n_head, D), np.float32)
    mp = 0
    if mask is not None:
        mask = np.ascontiguousarray(mask, dtype=np.uint16)
        mp = _p(mask)
    rc = lib().orc_flash_attn_ext(_p(q), _p(k), _p(v), mp or None, _p(out), D, n_q, n_head, n_kv, n_kv_head, scale,
                                  int(exact))
    if rc != 0:
        raise ValueError(f"orc_flash_attn_ext rc={rc}")
    return out


def fill_normal(seed: int, nrows: int, n_per_row: int, mean: float = 0.0, std: float = 1.0, row0: int = 0):
    out = np.empty((nrows, n_per_row), dtype=np.float32)
    lib().orc_fill_normal_rows(seed & 0xFFFFFFFFFFFFFFFF, row0, nrows, n_per_row, mean, std, _p(out))
    return out


def cpu_fast_mul_mat(wtype: int, w: np.ndarray, x: np.ndarray, nthreads: int) -> np.ndarray:
    """The AVX2 multi-threaded port of ggml's CPU mul_mat (x86 activation rounding)."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    N = w.shape[0]
    y = np.zeros((M, N), dtype=np.float32)
    s0, s1, d = _tensor(wtype, w, (K, N)), _tensor(TYPE_F32, x, (K, M)), _tensor(TYPE_F32, y, (N, M))
    rc = fast().cpf_mul_mat(ctypes.byref(s0), ctypes.byref(s1), ctypes.byref(d), int(nthreads))
    if rc != 0:
        raise ValueError(f"cpf_mul_mat rc={rc}")
    return y


def cpu_fast_flash_attn_ext(q: np.ndarray, k: np.ndarray, v: np.ndarray, mask, scale: float,
                            nthreads: int) -> np.ndarray:
    """The F16C multi-threaded port of ggml-cpu's flash attention over f16 K / V (the layouts of flash_attn_ext)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    n_head, n_q, D = q.shape
    n_kv_head, n_kv, _ = k.shape
    out = np.zeros((n_q, n_head, D), np.float32)
    mp = None
    if mask is not None:
        mask = np.ascontiguousarray(mask, dtype=np.uint16)
        mp = _p(mask)
    rc = fast().cpf_flash_attn_ext(_p(q), _p(k), _p(v), mp, _p(out), D, n_q, n_head, n_kv, n_kv_head, scale,
                                   int(nthreads))
    if rc != 0:
        raise ValueError(f"cpf_flash_attn_ext rc={rc}")
    return out


def physical_cores() -> int:
    """Physical core count (speech.cpp's default thread count, src/common/backend.cpp:122-167), capped by affinity."""
    try:
        seen = set()
        cpus = os.sched_getaffinity(0)
        for c in cpus:
            base = pathlib.Path(f"/sys/devices/system/cpu/cpu{c}/topology")
            core = (base / "core_id").read_text().strip()
            pkg = (base / "physical_package_id").read_text().strip()
            seen.add((pkg, core))
        return max(1, len(seen))
    except Exception:
        return max(1, (os.cpu_count() or 2) // 2)
