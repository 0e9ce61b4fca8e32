"""ctypes binding of librq (include/rq.h) with torch tensors for device memory.

torch is only plumbing here: it allocates device buffers and supplies the
current HIP stream; every kernel that runs is librq's.  The library must be
built (``python -m runtimed_amd.build``); a missing library raises, there is no
fallback path.
"""
from __future__ import annotations

import ctypes
from pathlib import Path
from typing import Optional

import numpy as np
import torch

LIB_PATH = Path(__file__).resolve().parent / "librq.so"

Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K = 2, 6, 8, 12, 13, 14
QTYPES = {"Q4_0": Q4_0, "Q5_0": Q5_0, "Q8_0": Q8_0, "Q4_K": Q4_K, "Q5_K": Q5_K, "Q6_K": Q6_K}
# (elements, bytes) per block, dtype.rs:49-64
GEOMETRY = {Q4_0: (32, 18), Q5_0: (32, 22), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176),
            Q6_K: (256, 210)}

F32, F16, BF16, F8E4M3 = 0, 1, 30, 128
FP8_UNSCALED, FP8_PER_TOKEN = 0, 1
_FTYPE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16, torch.float8_e4m3fn: F8E4M3,
          torch.uint8: F8E4M3}

STATUS = {0: "OK", -1: "Unsupported", -2: "Overflow", -3: "Truncated", -4: "Shape", -5: "Arg",
          -6: "Device", -7: "NoMem"}


class RqError(RuntimeError):
    """A negative rq_status with the library's thread-local message."""

    def __init__(self, code: int, message: str):
        super().__init__(f"{STATUS.get(code, code)}: {message}")
        self.code = code
        self.kind = STATUS.get(code, str(code))
        self.message = message


class _Desc(ctypes.Structure):
    _fields_ = [("qtype", ctypes.c_int32), ("device", ctypes.c_int32), ("n", ctypes.c_int64),
                ("k", ctypes.c_int64), ("gguf_bytes", ctypes.c_uint64),
                ("device_bytes", ctypes.c_uint64)]


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; run `python -m runtimed_amd.build`")
        L = ctypes.CDLL(str(LIB_PATH))
        vp, i64, sz, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_size_t, ctypes.c_int
        L.rq_abi_version.restype = i32
        L.rq_last_error.restype = ctypes.c_char_p
        L.rq_weight_create.argtypes = [i32, vp, sz, i64, i64, i32, ctypes.POINTER(vp)]
        L.rq_weight_destroy.argtypes = [vp]
        L.rq_weight_destroy.restype = None
        L.rq_weight_info.argtypes = [vp, ctypes.POINTER(_Desc)]
        L.rq_dequant_f32.argtypes = [vp, vp, vp]
        L.rq_dequant_tensor.argtypes = [i32, vp, sz, sz, vp, vp]
        L.rq_embedding.argtypes = [vp, vp, i64, vp, vp]
        L.rq_linear.argtypes = [vp, vp, i32, i64, vp, i32, vp]
        L.rq_fp8_quantize.argtypes = [vp, i32, i64, i64, i32, vp, vp, vp]
        L.rq_fp8_gemm.argtypes = [vp, i32, i64, vp, vp, i64, i64, vp, i32, i32, vp]
        L.rq_fp8_gemm_q.argtypes = [vp, vp, i64, vp, vp, i64, i64, vp, i32, vp]
        for f in ("rq_weight_create", "rq_weight_info", "rq_dequant_f32", "rq_dequant_tensor",
                  "rq_linear", "rq_fp8_quantize", "rq_fp8_gemm", "rq_fp8_gemm_q"):
            getattr(L, f).restype = i32
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        raise RqError(rc, lib().rq_last_error().decode())


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _ptr(t: Optional[torch.Tensor]) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


def ftype(dtype: torch.dtype) -> int:
    if dtype not in _FTYPE:
        raise TypeError(f"unsupported dtype {dtype}")
    return _FTYPE[dtype]


class QWeight:
    """A device-resident GGUF weight: the value a runtimed `q_map` entry holds.

    `blocks` is the GGUF block stream of an [n, k] tensor (GGUF dims [k, n]).
    """

    def __init__(self, qtype: int, blocks, n: int, k: int, device: int = 0):
        buf = np.ascontiguousarray(np.frombuffer(blocks, dtype=np.uint8)
                                   if not isinstance(blocks, np.ndarray) else blocks.view(np.uint8))
        h = ctypes.c_void_p()
        check(lib().rq_weight_create(qtype, buf.ctypes.data_as(ctypes.c_void_p), buf.nbytes, n, k,
                                     device, ctypes.byref(h)))
        self._h = h
        self.qtype, self.n, self.k, self.device = qtype, n, k, torch.device("cuda", device)

    def close(self) -> None:
        if getattr(self, "_h", None) and self._h.value:
            lib().rq_weight_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    def info(self) -> dict:
        d = _Desc()
        check(lib().rq_weight_info(self._h, ctypes.byref(d)))
        return {f: getattr(d, f) for f, _ in _Desc._fields_}

    def dequantize(self) -> torch.Tensor:
        out = torch.empty((self.n, self.k), dtype=torch.float32, device=self.device)
        check(lib().rq_dequant_f32(self._h, _ptr(out), _stream(self.device)))
        return out

    def embedding(self, ids) -> torch.Tensor:
        """Rows `ids` decoded exactly, f32 [len(ids), k] (embed_layer.rs:16-84)."""
        ids = np.ascontiguousarray(np.asarray(ids, dtype=np.uint32).reshape(-1))
        out = torch.empty((ids.size, self.k), dtype=torch.float32, device=self.device)
        check(lib().rq_embedding(self._h, ids.ctypes.data_as(ctypes.c_void_p), ids.size, _ptr(out),
                                 _stream(self.device)))
        return out

    def forward(self, x: torch.Tensor, out_dtype: Optional[torch.dtype] = None,
                out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """y = x W^T over the last dimension of x (linear_layer.rs:45-52)."""
        if x.shape[-1] != self.k:
            raise RqError(-4, f"expected last dim {self.k}, got {list(x.shape)}")
        if not x.is_contiguous():
            x = x.contiguous()
        rows = x.numel() // self.k if self.k else 0
        if out is None:
            out = torch.empty((*x.shape[:-1], self.n), dtype=out_dtype or x.dtype, device=x.device)
        check(lib().rq_linear(self._h, _ptr(x), ftype(x.dtype), rows, _ptr(out), ftype(out.dtype),
                              _stream(x.device)))
        return out


def dequant_tensor(qtype: int, dev_bytes: torch.Tensor, n_elements: int) -> torch.Tensor:
    """dequant_tensor (dequant.rs:83-146) on GGUF bytes in device memory."""
    out = torch.empty(n_elements, dtype=torch.float32, device=dev_bytes.device)
    check(lib().rq_dequant_tensor(qtype, _ptr(dev_bytes), dev_bytes.numel(), n_elements, _ptr(out),
                                  _stream(dev_bytes.device)))
    return out


def fp8_quantize(x: torch.Tensor, mode: int = FP8_PER_TOKEN):
    k = x.shape[-1]
    m = x.numel() // k
    xq = torch.empty((m, k), dtype=torch.uint8, device=x.device)
    xs = torch.empty(m, dtype=torch.float32, device=x.device)
    check(lib().rq_fp8_quantize(_ptr(x.contiguous()), ftype(x.dtype), m, k, mode, _ptr(xq), _ptr(xs),
                                _stream(x.device)))
    return xq, xs


def fp8_gemm(x: torch.Tensor, w: torch.Tensor, w_scale: Optional[torch.Tensor],
             mode: int = FP8_PER_TOKEN, out_dtype: torch.dtype = torch.bfloat16,
             out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = x (w * w_scale)^T with e4m3 w codes [n, k] (fp8_gemm.rs:77-191)."""
    n, k = w.shape
    if x.shape[-1] != k:
        raise RqError(-4, f"expected last dim {k}, got {list(x.shape)}")
    x = x.contiguous()
    m = x.numel() // k
    if out is None:
        out = torch.empty((*x.shape[:-1], n), dtype=out_dtype, device=x.device)
    check(lib().rq_fp8_gemm(_ptr(x), ftype(x.dtype), m, _ptr(w), _ptr(w_scale), n, k, _ptr(out),
                            ftype(out.dtype), mode, _stream(x.device)))
    return out


def fp8_gemm_q(xq: torch.Tensor, xs: Optional[torch.Tensor], w: torch.Tensor,
               w_scale: Optional[torch.Tensor], out: torch.Tensor) -> torch.Tensor:
    n, k = w.shape
    m = xq.numel() // k
    check(lib().rq_fp8_gemm_q(_ptr(xq), _ptr(xs), m, _ptr(w), _ptr(w_scale), n, k, _ptr(out),
                              ftype(out.dtype), _stream(xq.device)))
    return out
