"""ctypes view of the CPU oracle (oracle/librq_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by the smoke check of
__graft_entry__.py and by the CPU-baseline leg of bench.py, always to check
results or as the timed CPU baseline, never by the product path (runtimed_amd/).
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "librq_oracle.so"

OK, E_UNSUPPORTED, E_OVERFLOW, E_TRUNCATED = 0, -1, -2, -3
_lib = None


def build() -> Path:
    res = subprocess.run(["make", "-C", str(HERE), "-s"], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{res.stdout}\n{res.stderr}")
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        vp, i64, sz, u8, u16, u32, f32, i32 = (ctypes.c_void_p, ctypes.c_int64, ctypes.c_size_t,
                                               ctypes.c_uint8, ctypes.c_uint16, ctypes.c_uint32,
                                               ctypes.c_float, ctypes.c_int)
        L.rqo_block_geometry.argtypes = [u32, ctypes.POINTER(sz), ctypes.POINTER(sz)]
        L.rqo_f16_to_f32_bits.argtypes = [u16]
        L.rqo_f16_to_f32_bits.restype = u32
        for f in ("q8_0", "q4_0", "q5_0", "q4_k", "q5_k", "q6_k"):
            getattr(L, f"rqo_dequant_{f}_block").argtypes = [vp, vp]
        L.rqo_dequant_tensor.argtypes = [u32, vp, sz, sz, vp]
        L.rqo_dequant_tensor_mt.argtypes = [u32, vp, sz, sz, vp, i32]
        L.rqo_fp8_e4m3_to_f32.argtypes = [u8]
        L.rqo_fp8_e4m3_to_f32.restype = f32
        L.rqo_f32_to_fp8_e4m3.argtypes = [f32]
        L.rqo_f32_to_fp8_e4m3.restype = u8
        L.rqo_f32_to_fp8_e4m3_rne.argtypes = [f32]
        L.rqo_f32_to_fp8_e4m3_rne.restype = u8
        L.rqo_linear_f64.argtypes = [vp, i64, vp, i64, i64, vp]
        L.rqo_linear_f32.argtypes = [vp, i64, vp, i64, i64, vp, i32]
        L.rqo_fp8_gemm_fallback.argtypes = [vp, i64, vp, vp, i64, i64, vp]
        L.rqo_fp8_quantize_rows.argtypes = [vp, i64, i64, vp, vp]
        L.rqo_fp8_encode_unscaled.argtypes = [vp, i64, vp]
        L.rqo_fp8_gemm_quantized_f64.argtypes = [vp, vp, i64, vp, vp, i64, i64, vp]
        L.rqo_marlin_repack.argtypes = [vp, vp, i64, i64, vp]
        L.rqo_marlin_dequant.argtypes = [vp, vp, i64, i64, vp]
        L.rqo_marlin_gemv_f64.argtypes = [vp, i64, vp, vp, i64, i64, vp]
        L.rqo_kv_quantize.argtypes = [vp, i64, i64, i64, i32, vp, vp]
        L.rqo_kv_dequantize.argtypes = [vp, vp, i64, i64, i64, i32, vp]
        _lib = L
    return _lib


def _p(a: np.ndarray) -> ctypes.c_void_p:
    return a.ctypes.data_as(ctypes.c_void_p)


def geometry(dtype: int):
    e, b = ctypes.c_size_t(), ctypes.c_size_t()
    rc = lib().rqo_block_geometry(dtype, ctypes.byref(e), ctypes.byref(b))
    return (e.value, b.value) if rc == OK else None


def f16_to_f32_bits(h: int) -> int:
    return lib().rqo_f16_to_f32_bits(h)


def dequant_block(kind: str, block) -> np.ndarray:
    blk = np.ascontiguousarray(np.frombuffer(bytes(block), dtype=np.uint8))
    out = np.zeros(256 if kind.endswith("_k") else 32, dtype=np.float32)
    getattr(lib(), f"rqo_dequant_{kind}_block")(_p(blk), _p(out))
    return out


def dequant_tensor(dtype: int, data: np.ndarray, n_elements: int, threads: int = 1):
    """(status, f32 array) -- dequant_tensor semantics (dequant.rs:83-146)."""
    data = np.ascontiguousarray(data, dtype=np.uint8)
    out = np.empty(max(n_elements, 1), dtype=np.float32)
    if threads > 1:
        rc = lib().rqo_dequant_tensor_mt(dtype, _p(data), data.nbytes, n_elements, _p(out), threads)
    else:
        rc = lib().rqo_dequant_tensor(dtype, _p(data), data.nbytes, n_elements, _p(out))
    return rc, out[:n_elements]


def fp8_decode(b: int) -> float:
    return lib().rqo_fp8_e4m3_to_f32(b)


def fp8_encode(f: float) -> int:
    return lib().rqo_f32_to_fp8_e4m3(f)


def fp8_encode_rne(f: float) -> int:
    return lib().rqo_f32_to_fp8_e4m3_rne(f)


def fp8_encode_array(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint8)
    lib().rqo_fp8_encode_unscaled(_p(x), x.size, _p(out))
    return out


def linear_f64(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    m, k = x.shape
    n = w.shape[0]
    y = np.empty((m, n), dtype=np.float64)
    lib().rqo_linear_f64(_p(x), m, _p(w), n, k, _p(y))
    return y


def linear_f32(x: np.ndarray, w: np.ndarray, threads: int = 1) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    m, k = x.shape
    n = w.shape[0]
    y = np.empty((m, n), dtype=np.float32)
    lib().rqo_linear_f32(_p(x), m, _p(w), n, k, _p(y), threads)
    return y


def fp8_gemm_fallback(x: np.ndarray, w_codes: np.ndarray, scale: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w_codes = np.ascontiguousarray(w_codes, dtype=np.uint8)
    scale = np.ascontiguousarray(scale, dtype=np.float32)
    m, k = x.shape
    n = w_codes.shape[0]
    y = np.empty((m, n), dtype=np.float32)
    lib().rqo_fp8_gemm_fallback(_p(x), m, _p(w_codes), _p(scale), n, k, _p(y))
    return y


def fp8_quantize_rows(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, k = x.shape
    xq = np.empty((m, k), dtype=np.uint8)
    xs = np.empty(m, dtype=np.float32)
    lib().rqo_fp8_quantize_rows(_p(x), m, k, _p(xq), _p(xs))
    return xq, xs


def fp8_gemm_quantized_f64(xq, xs, w_codes, ws) -> np.ndarray:
    xq = np.ascontiguousarray(xq, dtype=np.uint8)
    xs = np.ascontiguousarray(xs, dtype=np.float32)
    w_codes = np.ascontiguousarray(w_codes, dtype=np.uint8)
    ws = np.ascontiguousarray(ws, dtype=np.float32)
    m, k = xq.shape
    n = w_codes.shape[0]
    y = np.empty((m, n), dtype=np.float64)
    lib().rqo_fp8_gemm_quantized_f64(_p(xq), _p(xs), m, _p(w_codes), _p(ws), n, k, _p(y))
    return y


# ---- Marlin INT4 weights (marlin_gemv.rs) ----

def marlin_repack(w: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """repack_marlin_tiles (marlin_gemv.rs:66-97): u32 [ceil(k/32), n, 4]."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    scales = np.ascontiguousarray(scales, dtype=np.float32).reshape(-1)
    n, k = w.shape
    packed = np.empty(((k + 31) // 32, n, 4), dtype=np.uint32)
    lib().rqo_marlin_repack(_p(w), _p(scales), n, k, _p(packed))
    return packed


def marlin_dequant(packed: np.ndarray, scales: np.ndarray, k: int) -> np.ndarray:
    """MarlinWeight::dequantize (marlin_gemv.rs:42-61): f32 [n, k]."""
    packed = np.ascontiguousarray(packed, dtype=np.uint32)
    scales = np.ascontiguousarray(scales, dtype=np.float32).reshape(-1)
    n = scales.size
    out = np.empty((n, k), dtype=np.float32)
    lib().rqo_marlin_dequant(_p(packed), _p(scales), n, k, _p(out))
    return out


def marlin_gemv_f64(x: np.ndarray, packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    packed = np.ascontiguousarray(packed, dtype=np.uint32)
    scales = np.ascontiguousarray(scales, dtype=np.float32).reshape(-1)
    m, k = x.shape
    n = scales.size
    y = np.empty((m, n), dtype=np.float64)
    lib().rqo_marlin_gemv_f64(_p(x), m, _p(packed), _p(scales), n, k, _p(y))
    return y


# ---- paged-KV quantizer (cache/paged/quantize.rs) ----

def kv_quantize(t: np.ndarray, int8: bool = False):
    """quantize_fp8 / quantize_int8 (quantize.rs:12-46, 62-96): (codes u8 of
    t's shape, scales f32 [h]); a tensor that is not 4-D counts as [1, 1, n, 1]."""
    t = np.ascontiguousarray(t, dtype=np.float32)
    b, h, sd = (t.shape[0], t.shape[1], t.shape[2] * t.shape[3]) if t.ndim == 4 else (1, 1, t.size)
    q = np.empty(t.shape, dtype=np.uint8)
    s = np.empty(h, dtype=np.float32)
    lib().rqo_kv_quantize(_p(t), b, h, sd, int(int8), _p(q), _p(s))
    return q, s


def kv_dequantize(q: np.ndarray, scales: np.ndarray, int8: bool = False) -> np.ndarray:
    """dequantize_fp8 / dequantize_int8 (quantize.rs:48-57, 98-107) in f32."""
    q = np.ascontiguousarray(q, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32).reshape(-1)
    b, h, sd = (q.shape[0], q.shape[1], q.shape[2] * q.shape[3]) if q.ndim == 4 else (1, 1, q.size)
    out = np.empty(q.shape, dtype=np.float32)
    lib().rqo_kv_dequantize(_p(q), _p(scales), b, h, sd, int(int8), _p(out))
    return out
