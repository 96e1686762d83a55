"""Shared helpers of the parity tests."""
import numpy as np


def rel_err(y: np.ndarray, y_ref: np.ndarray) -> float:
    """Largest |y - y_ref| of each output row over the largest |y_ref| of that row, maximised over rows.

    A row is one src1 column's outputs (ne0 of dst). This is the 'max relative error' the parity bar is stated in."""
    y = np.asarray(y, dtype=np.float64).reshape(-1, y_ref.shape[-1])
    r = np.asarray(y_ref, dtype=np.float64).reshape(-1, y_ref.shape[-1])
    scale = np.maximum(np.abs(r).max(axis=1), 1e-30)
    return float((np.abs(y - r).max(axis=1) / scale).max())


def l2_rel(y: np.ndarray, y_ref: np.ndarray) -> float:
    """Row-relative L2 error, as speech.cpp's decoder check measures it (checks/common/qwen3-decoder-check.cpp:59-66)."""
    y = np.asarray(y, dtype=np.float64).reshape(-1, y_ref.shape[-1])
    r = np.asarray(y_ref, dtype=np.float64).reshape(-1, y_ref.shape[-1])
    return float((np.linalg.norm(y - r, axis=1) / np.maximum(np.linalg.norm(r, axis=1), 1e-30)).max())


def bits_equal(a: np.ndarray, b: np.ndarray) -> bool:
    return a.shape == b.shape and np.array_equal(np.ascontiguousarray(a).view(np.uint8),
                                                 np.ascontiguousarray(b).view(np.uint8))


def dq_row_exp(amax: np.ndarray) -> np.ndarray:
    """The power of two the fp16 GEMM scales an activation row by: 2^e puts the row's largest |value| in
    [2^14, 2^15) (e = 0 for an all-zero row; e within [-126, 126], so 2^-e is a normal float)."""
    _, ex = np.frexp(amax.astype(np.float64))  # amax = f 2^ex, f in [0.5, 1)
    e = np.where(amax > 0, 15 - ex, 0)
    return np.clip(e, -126, 126)


def dq_model(oracle, wtype: int, w: np.ndarray, x: np.ndarray, K: int, rounding: int = 0) -> np.ndarray:
    """What the dequantizing fp16 GEMM computes, exactly up to its fp32 summation order: every weight and every
    quantized activation (the oracle's own quantization of x for the weight's dot, its fp32 values times the row's
    power-of-two scale) rounded once to fp16, products summed in float64 and the scale taken off. Kernel against this
    model: ~1e-6; this model against the oracle: a few 1e-4."""
    act_type = oracle.TYPE_Q8_0 if wtype == oracle.TYPE_Q8_0 else oracle.TYPE_Q8_K
    wd = oracle.dequantize_rows(wtype, w, K).astype(np.float16).astype(np.float64)
    xq = oracle.quantize_rows(act_type, np.ascontiguousarray(x, dtype=np.float32), rounding)
    xv = oracle.dequantize_rows(act_type, xq, K).astype(np.float64)
    sc = np.ldexp(1.0, dq_row_exp(np.abs(xv).max(axis=1)))[:, None]
    xd = (xv * sc).astype(np.float16).astype(np.float64) / sc
    return xd @ wd.T
